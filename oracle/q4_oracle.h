/*
 * q4_oracle.h -- CPU oracle for the W4A8 projections on either side of the
 * attention step (Q4_0 weights x Q8_0 activations).
 *
 * TEST INFRASTRUCTURE ONLY, like miattn_oracle.h: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Block formats (mistral/dequant.h):
 *   Q4_0  18 bytes per 32 weights: fp16 scale d, then 16 bytes whose low
 *         nibbles are weights 0..15 and high nibbles weights 16..31, each
 *         stored + 8 (dequant.h:14-21, 600-611)
 *   Q8_0  36 bytes per 32 values: fp32 scale d, then 32 int8 (dequant.h:535-541)
 *
 * Pinning status (tests/test_oracle_q4.py):
 *   ora_quantize_q8_0      known answers (scale, ties to even, zero block,
 *                          saturation bound), and |x - d*q| <= d/2        pinned
 *   ora_q4_0_q8_0_matvec   every block's integer dot against a brute-force
 *                          int64 sum; the whole product against float64
 *                          dequantised weights x activations              pinned
 *   ora_q4_0_q8_0_matvec_qkv  == three ora_q4_0_q8_0_matvec calls         pinned
 * The fp32 order of the block sums follows the reference's sequential loop;
 * whether the reference's compiler contracts `sum += (wd*xd)*isum` into an
 * fma is not fixed by any test there (parity unpinned at the ulp level).
 */
#ifndef Q4_ORACLE_H
#define Q4_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORA_QK 32

typedef struct {
    float d;
    int8_t qs[ORA_QK];
} OraQ8Block;  /* 36 bytes, mistral/dequant.h:537-541 */

/* mistral/dequant.h:545-612: n a multiple of 32 */
void ora_quantize_q8_0(const float *x, OraQ8Block *out, int n);

/* y[out_dim] = W[out_dim][in_dim] (Q4_0 rows, 18 B per block) . x (Q8_0),
 * the arithmetic of mistral/dequant.h:1022-1137 (q4_0_q8_0_matvec_sdot_parallel,
 * the path mistral_model.h:649-655 takes for Q4_0 with out_dim >= 128). */
void ora_q4_0_q8_0_matvec(const void *W, const OraQ8Block *x, float *y, int out_dim, int in_dim);

/* mistral_model.h:676-745: Q, K and V rows against one quantised input. */
void ora_q4_0_q8_0_matvec_qkv(const void *Wq, const void *Wk, const void *Wv,
                              const OraQ8Block *x, float *yq, float *yk, float *yv, int dim,
                              int kv_dim, int in_dim);

/* Timing (CPU baseline): rows over OpenMP threads, same arithmetic. */
void ora_q4_0_q8_0_matvec_parallel(const void *W, const OraQ8Block *x, float *y, int out_dim,
                                   int in_dim, int threads);

#ifdef __cplusplus
}
#endif

#endif
