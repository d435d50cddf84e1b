/*
 * q4_oracle.c -- CPU oracle for the Q4_0 x Q8_0 projections (test
 * infrastructure only; see q4_oracle.h).
 *
 * Scalar restatement of mistral/dequant.h's W4A8 path.  Substitutions:
 *   vabsq / vmaxq / vmaxvq            -> fabsf / fmaxf loop (order-free)
 *   vcvtnq_s32_f32 (ties to even)     -> nearbyintf in the default rounding mode
 *   vqmovn_s32 then vqmovn_s16        -> clamp to [-128, 127]
 *   vdotq_s32 + vaddvq_s32            -> int32 loop (exact: |sum| < 2^18)
 */
#include "q4_oracle.h"

#include <math.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static float f16_bits_to_f32(uint16_t h) {
    const uint32_t s = (uint32_t)(h >> 15) << 31, e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = s;
        } else { /* subnormal: value m * 2^-24 */
            float v = (float)m * 5.9604644775390625e-8f;
            memcpy(&bits, &v, 4);
            bits |= s;
        }
    } else if (e == 31) {
        bits = s | 0x7f800000u | (m << 13);
    } else {
        bits = s | ((e + 112) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* mistral/dequant.h:545-612 */
void ora_quantize_q8_0(const float *x, OraQ8Block *out, int n) {
    const int nb = n / ORA_QK;
    for (int i = 0; i < nb; i++) {
        const float *src = x + i * ORA_QK;
        float amax = 0.0f;
        for (int j = 0; j < ORA_QK; j++) amax = fmaxf(amax, fabsf(src[j]));
        const float d = amax / 127.0f;
        out[i].d = d;
        if (amax == 0.0f) {
            memset(out[i].qs, 0, ORA_QK);
            continue;
        }
        const float id = 1.0f / d;
        for (int j = 0; j < ORA_QK; j++) {
            float r = nearbyintf(src[j] * id);
            if (r > 127.0f) r = 127.0f;
            if (r < -128.0f) r = -128.0f;
            out[i].qs[j] = (int8_t)r;
        }
    }
}

/* One row: sequential sum over the blocks of (wd * xd) * isum
 * (mistral/dequant.h:1070-1087, 1093-1118). */
static float q4_row(const uint8_t *row, const OraQ8Block *x, int bpr) {
    float sumf = 0.0f;
    for (int b = 0; b < bpr; b++) {
        const uint8_t *blk = row + (size_t)b * 18;
        const float wd = f16_bits_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
        const float xd = x[b].d;
        int32_t isum = 0;
        for (int j = 0; j < 16; j++) {
            const int lo = (int)(blk[2 + j] & 0x0f) - 8; /* weight j */
            const int hi = (int)(blk[2 + j] >> 4) - 8;   /* weight j + 16 */
            isum += lo * x[b].qs[j] + hi * x[b].qs[j + 16];
        }
        sumf += (wd * xd) * (float)isum;
    }
    return sumf;
}

void ora_q4_0_q8_0_matvec(const void *W, const OraQ8Block *x, float *y, int out_dim, int in_dim) {
    const int bpr = in_dim / ORA_QK;
    const uint8_t *w = (const uint8_t *)W;
    for (int r = 0; r < out_dim; r++) y[r] = q4_row(w + (size_t)r * bpr * 18, x, bpr);
}

/* mistral_model.h:676-745: virtual rows 0..dim-1 are Wq, then Wk, then Wv. */
void ora_q4_0_q8_0_matvec_qkv(const void *Wq, const void *Wk, const void *Wv,
                              const OraQ8Block *x, float *yq, float *yk, float *yv, int dim,
                              int kv_dim, int in_dim) {
    ora_q4_0_q8_0_matvec(Wq, x, yq, dim, in_dim);
    ora_q4_0_q8_0_matvec(Wk, x, yk, kv_dim, in_dim);
    ora_q4_0_q8_0_matvec(Wv, x, yv, kv_dim, in_dim);
}

void ora_q4_0_q8_0_matvec_parallel(const void *W, const OraQ8Block *x, float *y, int out_dim,
                                   int in_dim, int threads) {
    const int bpr = in_dim / ORA_QK;
    const uint8_t *w = (const uint8_t *)W;
#ifdef _OPENMP
    if (threads <= 0) threads = omp_get_max_threads();
#pragma omp parallel for schedule(static) num_threads(threads)
#else
    (void)threads;
#endif
    for (int r = 0; r < out_dim; r++) y[r] = q4_row(w + (size_t)r * bpr * 18, x, bpr);
}
