/*
 * kquant_oracle.c -- CPU oracle for the Q4_K / Q6_K / F16 / F32 weight paths
 * (test infrastructure only; see kquant_oracle.h).
 *
 * Scalar restatement.  Substitutions:
 *   vmulq_f16 / vsubq_f16 (fp16 RNE)   -> exact product / difference in double,
 *                                          one round to fp16 (RNE, subnormals)
 *   (_Float16)(float)                  -> the same rounding from the exact value
 *   vfmaq_f32 lanes + vaddvq_f32       -> fmaf into four lane sums, then
 *                                          (l0 + l1) + (l2 + l3)
 *   cblas_sgemv / cblas_sgemm          -> fp32 sums in k order
 */
#include "kquant_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include "prefill_oracle.h"
#ifdef _OPENMP
#include <omp.h>
#endif

#define QK_K 256

/* fp16 bits nearest to v (RNE), v exactly representable in double: the
 * value of one IEEE binary16 operation on binary16 operands. */
static uint16_t f16_round(double v) {
    uint16_t sign = 0;
    if (v < 0 || (v == 0 && signbit(v))) {
        sign = 0x8000;
        v = -v;
    }
    if (isnan(v)) return 0x7e00;
    if (v >= 65520.0) return sign | 0x7c00; /* rounds to infinity */
    if (v < 6.103515625e-05) {              /* below 2^-14: subnormal grid 2^-24 */
        const double m = nearbyint(v * 16777216.0);
        return sign | (uint16_t)m; /* m == 1024 is the smallest normal: same bits */
    }
    int e;
    const double f = frexp(v, &e); /* v = f * 2^e, f in [0.5, 1) */
    double m = nearbyint(f * 2048.0); /* 11 significant bits */
    if (m == 2048.0) {
        m = 1024.0;
        e += 1;
    }
    if (e + 14 >= 31) return sign | 0x7c00;
    return sign | (uint16_t)((e + 14) << 10) | (uint16_t)((int)m - 1024);
}

long ora_typed_row_bytes(int type, int cols) {
    switch (type) {
    case ORA_TYPE_F32: return (long)cols * 4;
    case ORA_TYPE_F16: return (long)cols * 2;
    case ORA_TYPE_Q4_0: return cols % 32 ? 0 : (long)(cols / 32) * 18;
    case ORA_TYPE_Q4_K: return cols % QK_K ? 0 : (long)(cols / QK_K) * 144;
    case ORA_TYPE_Q6_K: return cols % QK_K ? 0 : (long)(cols / QK_K) * 210;
    default: return 0;
    }
}

/* mistral/dequant.h:58-66 */
static void scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

/* mistral/dequant.h:68-125: 64 values per pass, the low nibbles of 32 bytes
 * with sub-block scale/min (is), the high nibbles with (is + 1); every step
 * in fp16: (_Float16)(d * sc), q * that, minus (_Float16)(dmin * m). */
static void dequant_q4_k_block(const uint8_t *blk, float *out) {
    uint16_t dh, mh;
    memcpy(&dh, blk, 2);
    memcpy(&mh, blk + 2, 2);
    const float d = ora_f16_to_f32(dh), dmin = ora_f16_to_f32(mh);
    const uint8_t *scales = blk + 4, *qs = blk + 16;
    for (int j = 0, is = 0; j < QK_K; j += 64, is += 2, qs += 32) {
        uint8_t sc1, m1, sc2, m2;
        scale_min_k4(is, scales, &sc1, &m1);
        scale_min_k4(is + 1, scales, &sc2, &m2);
        /* d * sc (an 11-bit significand times a 6-bit integer) is exact in
         * fp32 and double alike */
        const double vd1 = ora_f16_to_f32(f16_round((double)d * sc1));
        const double vm1 = ora_f16_to_f32(f16_round((double)dmin * m1));
        const double vd2 = ora_f16_to_f32(f16_round((double)d * sc2));
        const double vm2 = ora_f16_to_f32(f16_round((double)dmin * m2));
        for (int l = 0; l < 32; l++) {
            const double p1 = ora_f16_to_f32(f16_round((double)(qs[l] & 0x0F) * vd1));
            const double p2 = ora_f16_to_f32(f16_round((double)(qs[l] >> 4) * vd2));
            out[j + l] = ora_f16_to_f32(f16_round(p1 - vm1));
            out[j + 32 + l] = ora_f16_to_f32(f16_round(p2 - vm2));
        }
    }
}

/* mistral/dequant.h:291-307: value n from ql[n % 128] (low nibble below 128,
 * high nibble from 128) and the 2-bit field of qh[n % 64] at bit
 * 2 * (n / 128) + 4 * (n % 128 >= 64); weight = d * scales[n / 16] * q, q in
 * [-32, 31], multiplied left to right in fp32. */
static void dequant_q6_k_block(const uint8_t *blk, float *out) {
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t *sc = (const int8_t *)(blk + 192);
    uint16_t dh;
    memcpy(&dh, blk + 208, 2);
    const float d = ora_f16_to_f32(dh);
    for (int n = 0; n < QK_K; n++) {
        const int il = n % 128, is = n / 16, ih = n / 128;
        const uint8_t q_lo = n < 128 ? (ql[il] & 0xF) : (ql[il] >> 4);
        const uint8_t q_hi = (qh[il % 64] >> (2 * ih + (il >= 64 ? 4 : 0))) & 3;
        const int8_t q = (int8_t)((q_lo | (q_hi << 4)) - 32);
        out[n] = d * sc[is] * q;
    }
}

int ora_dequant_typed_rows(const void *W, int type, float *dst, int rows, int cols) {
    const long rb = ora_typed_row_bytes(type, cols);
    if (rb == 0) return -1;
    for (int r = 0; r < rows; r++) {
        const uint8_t *row = (const uint8_t *)W + (size_t)r * rb;
        float *o = dst + (size_t)r * cols;
        switch (type) {
        case ORA_TYPE_F32: memcpy(o, row, (size_t)cols * 4); break;
        case ORA_TYPE_F16:
            for (int i = 0; i < cols; i++) {
                uint16_t h;
                memcpy(&h, row + 2 * i, 2);
                o[i] = ora_f16_to_f32(h);
            }
            break;
        case ORA_TYPE_Q4_0: /* mistral_ane_prefill.h:921-939 */
            for (int b = 0; b < cols / 32; b++) {
                const uint8_t *blk = row + 18 * b;
                uint16_t dh;
                memcpy(&dh, blk, 2);
                const float d = ora_f16_to_f32(dh);
                for (int i = 0; i < 16; i++) {
                    o[32 * b + i] = d * ((float)(blk[2 + i] & 0x0F) - 8.0f);
                    o[32 * b + i + 16] = d * ((float)(blk[2 + i] >> 4) - 8.0f);
                }
            }
            break;
        case ORA_TYPE_Q4_K:
            for (int b = 0; b < cols / QK_K; b++) dequant_q4_k_block(row + 144 * b, o + QK_K * b);
            break;
        case ORA_TYPE_Q6_K:
            for (int b = 0; b < cols / QK_K; b++) dequant_q6_k_block(row + 210 * b, o + QK_K * b);
            break;
        default: return -1;
        }
    }
    return 0;
}

int ora_typed_matvec(const void *W, int type, const float *x, float *y, int out_dim, int in_dim) {
    const long rb = ora_typed_row_bytes(type, in_dim);
    if (rb == 0) return -1;
    float tmp[QK_K];
    for (int r = 0; r < out_dim; r++) {
        const uint8_t *row = (const uint8_t *)W + (size_t)r * rb;
        if (type == ORA_TYPE_Q4_0) {
            /* q4_0_matvec_f32 (dequant.h:142-278): w = (q - 8) * d in fp32,
             * lane l of four accumulating values 4k + l with fma; vaddvq */
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            for (int b = 0; b < in_dim / 32; b++) {
                ora_dequant_typed_rows(row + 18 * b, ORA_TYPE_Q4_0, tmp, 1, 32);
                for (int i = 0; i < 32; i++)
                    acc[i & 3] = fmaf(tmp[i], x[32 * b + i], acc[i & 3]);
            }
            y[r] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        } else if (type == ORA_TYPE_Q6_K) {
            /* dequant.h:365-521: lane l accumulates values 4k + l of the row
             * with fma, sub-block after sub-block; then vaddvq */
            float acc[4] = {0.f, 0.f, 0.f, 0.f};
            for (int b = 0; b < in_dim / QK_K; b++) {
                dequant_q6_k_block(row + 210 * b, tmp);
                for (int i = 0; i < QK_K; i++)
                    acc[i & 3] = fmaf(tmp[i], x[QK_K * b + i], acc[i & 3]);
            }
            y[r] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
        } else {
            float sum = 0.f;
            for (int c0 = 0; c0 < in_dim; c0 += QK_K) {
                const int n = in_dim - c0 < QK_K ? in_dim - c0 : QK_K;
                if (type == ORA_TYPE_Q4_K) {
                    dequant_q4_k_block(row + 144 * (c0 / QK_K), tmp);
                } else if (type == ORA_TYPE_F16) {
                    for (int i = 0; i < n; i++) {
                        uint16_t h;
                        memcpy(&h, row + 2 * (c0 + i), 2);
                        tmp[i] = ora_f16_to_f32(h);
                    }
                } else {
                    memcpy(tmp, row + 4 * (size_t)c0, (size_t)n * 4);
                }
                for (int i = 0; i < n; i++) sum += tmp[i] * x[c0 + i];
            }
            y[r] = sum;
        }
    }
    return 0;
}

int ora_typed_matvec_q8(const void *W, int type, const OraQ8Block *xq, float *y, int out_dim,
                        int in_dim) {
    if (in_dim % ORA_QK) return -1;
    float *x = (float *)__builtin_alloca((size_t)in_dim * sizeof(float));
    for (int b = 0; b < in_dim / ORA_QK; b++)
        for (int j = 0; j < ORA_QK; j++) x[b * ORA_QK + j] = xq[b].d * xq[b].qs[j];
    return ora_typed_matvec(W, type, x, y, out_dim, in_dim);
}

int ora_typed_gemm(const void *W, int type, int out_dim, int in_dim, const float *X, int S,
                   float *Y, int threads) {
    const long rb = ora_typed_row_bytes(type, in_dim);
    if (rb == 0) return -1;
    int bad = 0;
#ifdef _OPENMP
    const int nt = threads > 0 ? threads : omp_get_max_threads();
#pragma omp parallel for num_threads(nt) schedule(dynamic, 8) reduction(| : bad)
#else
    (void)threads;
#endif
    for (int n = 0; n < out_dim; n++) {
        float w[in_dim];
        bad |= ora_dequant_typed_rows((const uint8_t *)W + (size_t)n * rb, type, w, 1, in_dim) != 0;
        for (int t = 0; t < S; t++) {
            const float *xr = X + (size_t)t * in_dim;
            float sum = 0.f;
            for (int k = 0; k < in_dim; k++) sum += xr[k] * w[k];
            Y[(size_t)t * out_dim + n] = sum;
        }
    }
    return bad ? -1 : 0;
}

int ora_prefill_layer_typed(const OraLayerWeightsTyped *lw, OraKV *kv, float *X, int layer,
                            int start_pos, int S, int dim, int hidden, int n_heads,
                            int n_kv_heads, float eps, const float *theta_inv, int threads) {
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
    int bad = 0;
    /* mistral_ane_prefill.h:1092-1110 */
    ora_rmsnorm_batch(Xn, X, lw->rms_att, dim, S, eps);
    bad |= ora_typed_gemm(lw->wq, lw->wq_type, dim, dim, Xn, S, Q, threads);
    bad |= ora_typed_gemm(lw->wk, lw->wk_type, kv_dim, dim, Xn, S, K, threads);
    bad |= ora_typed_gemm(lw->wv, lw->wv_type, kv_dim, dim, Xn, S, V, threads);
    ora_apply_rope_batch(Q, K, start_pos, theta_inv, n_heads, n_kv_heads, hd, S);
    ora_kv_write_batch(kv, layer, start_pos, K, V, kv_dim, S);
    ora_attention_batch(Q, A, kv, layer, start_pos, n_heads, n_kv_heads, hd, S, att);
    bad |= ora_typed_gemm(lw->wo, lw->wo_type, dim, dim, A, S, Xn, threads);
    for (size_t i = 0; i < sd; i++) X[i] = X[i] + Xn[i];
    ora_rmsnorm_batch(Xn, X, lw->rms_ffn, dim, S, eps);
    bad |= ora_typed_gemm(lw->w1, lw->w1_type, hidden, dim, Xn, S, G, threads);
    bad |= ora_typed_gemm(lw->w3, lw->w3_type, hidden, dim, Xn, S, U, threads);
    ora_silu_mul(G, U, (int)sh);
    bad |= ora_typed_gemm(lw->w2, lw->w2_type, dim, hidden, G, S, Xn, threads);
    for (size_t i = 0; i < sd; i++) X[i] = X[i] + Xn[i];
    free(Xn); free(Q); free(K); free(V); free(A); free(G); free(U); free(att);
    return bad ? -1 : 0;
}

/* y = W . x_q8 by type, as q4_matvec_sdot_parallel dispatches
 * (mistral_model.h:649-670) */
static int layer_matvec(const void *W, int type, const OraQ8Block *xq, float *y, int rows,
                        int cols) {
    if (type == ORA_TYPE_Q4_0) {
        ora_q4_0_q8_0_matvec(W, xq, y, rows, cols);
        return 0;
    }
    return ora_typed_matvec_q8(W, type, xq, y, rows, cols);
}

int ora_decode_layer_typed(const OraLayerWeightsTyped *lw, OraKV *kv, float *x, int layer,
                           int pos, int dim, int hidden, int n_heads, int n_kv_heads, float eps,
                           const float *theta_inv) {
    const int kv_dim = n_kv_heads * (dim / n_heads);
    float *xb = (float *)malloc((size_t)dim * sizeof(float));
    float *xb2 = (float *)malloc((size_t)dim * sizeof(float));
    float *q = (float *)malloc((size_t)dim * sizeof(float));
    float *k = (float *)malloc((size_t)kv_dim * sizeof(float));
    float *v = (float *)malloc((size_t)kv_dim * sizeof(float));
    float *hb = (float *)malloc((size_t)hidden * sizeof(float));
    float *hb2 = (float *)malloc((size_t)hidden * sizeof(float));
    float *att = (float *)malloc((size_t)n_heads * kv->max_seq * sizeof(float));
    OraQ8Block *xq = (OraQ8Block *)malloc((size_t)(dim > hidden ? dim : hidden) / ORA_QK *
                                          sizeof(OraQ8Block));
    if (!xb || !xb2 || !q || !k || !v || !hb || !hb2 || !att || !xq) abort();
    int bad = 0;
    /* mistral_model.h:830-899 */
    ora_rmsnorm_batch(xb, x, lw->rms_att, dim, 1, eps);
    ora_quantize_q8_0(xb, xq, dim);
    bad |= layer_matvec(lw->wq, lw->wq_type, xq, q, dim, dim);
    bad |= layer_matvec(lw->wk, lw->wk_type, xq, k, kv_dim, dim);
    bad |= layer_matvec(lw->wv, lw->wv_type, xq, v, kv_dim, dim);
    ora_decode_step(kv, layer, q, k, v, pos, theta_inv, n_heads, n_kv_heads, att, xb2);
    ora_quantize_q8_0(xb2, xq, dim);
    bad |= layer_matvec(lw->wo, lw->wo_type, xq, xb, dim, dim);
    for (int i = 0; i < dim; i++) x[i] = x[i] + xb[i];
    ora_rmsnorm_batch(xb, x, lw->rms_ffn, dim, 1, eps);
    ora_quantize_q8_0(xb, xq, dim);
    bad |= layer_matvec(lw->w1, lw->w1_type, xq, hb, hidden, dim);
    bad |= layer_matvec(lw->w3, lw->w3_type, xq, hb2, hidden, dim);
    ora_silu_mul(hb, hb2, hidden);
    ora_quantize_q8_0(hb, xq, hidden);
    bad |= layer_matvec(lw->w2, lw->w2_type, xq, xb, dim, hidden);
    for (int i = 0; i < dim; i++) x[i] = x[i] + xb[i];
    free(xb); free(xb2); free(q); free(k); free(v); free(hb); free(hb2); free(att); free(xq);
    return bad ? -1 : 0;
}
