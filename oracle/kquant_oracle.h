/*
 * kquant_oracle.h -- CPU oracle for the weight types other than Q4_0 that the
 * reference's projections and prefill GEMM accept: Q4_K and Q6_K (the
 * Q4_K_M GGUF files it targets), F16 and F32.
 *
 * TEST INFRASTRUCTURE ONLY, like miattn_oracle.h: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Block formats (mistral/dequant.h):
 *   Q4_K  144 bytes per 256 weights: fp16 d, fp16 dmin, 12 bytes of packed
 *         6-bit sub-block scales and mins, 128 bytes of nibbles
 *         (dequant.h:23-29, 58-66)
 *   Q6_K  210 bytes per 256 weights: ql[128] low nibbles, qh[64] high bit
 *         pairs, int8 scales[16], fp16 d (dequant.h:283-289)
 *
 * Pinning status (tests/test_oracle_kquant.py):
 *   ora_dequant_typed_rows  Q4_K: known answers for every sub-block's scale
 *                           and min (both branches of get_scale_min_k4) and
 *                           the nibble order, and a numpy restatement of the
 *                           reference's fp16 arithmetic (each step rounded
 *                           from float64 to fp16); Q6_K: single-value blocks
 *                           reveal the value mapping of every position, and
 *                           a float64 restatement; F16 / F32 exact     pinned
 *   ora_typed_matvec        float64 dot of the dequantised rows (the
 *                           reference's sgemv order is BLAS's: parity
 *                           unpinned at the ulp level); Q6_K follows the
 *                           reference's four-lane fma order        pinned
 *   ora_typed_matvec_q8     == ora_typed_matvec on the Q8_0 values  pinned
 *   ora_typed_gemm          float64 matmul of the dequantised rows; the
 *                           Q4_0 branch equals prefill_oracle's GEMM  pinned
 *   ora_prefill_layer_typed all-Q4_0 weights reproduce ora_prefill_layer
 *                           bit for bit; its other steps are that
 *                           function's (prefill_oracle.h)            pinned
 *   ora_decode_layer_typed  against a float64 numpy layer on the oracle's
 *                           own Q8_0 activations                     pinned
 */
#ifndef KQUANT_ORACLE_H
#define KQUANT_ORACLE_H

#include <stdint.h>

#include "miattn_oracle.h"
#include "q4_oracle.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids (mistral/gguf_loader.h:32-38) */
enum { ORA_TYPE_F32 = 0, ORA_TYPE_F16 = 1, ORA_TYPE_Q4_0 = 2, ORA_TYPE_Q4_K = 12, ORA_TYPE_Q6_K = 14 };

/* Bytes of one row of `cols` weights of the type (0: unsupported type or
 * cols not a multiple of the block); mistral_ane_prefill.h:1008-1015. */
long ora_typed_row_bytes(int type, int cols);

/* The fp32 weights the reference multiplies (dequant_weight_to_fp32_buf,
 * mistral_ane_prefill.h:907-1000; q4_matvec's Q4_K branch,
 * mistral_model.h:215-226, yields the same values): Q4_K through the fp16
 * arithmetic of dequant_q4_K_block_neon (dequant.h:68-125), Q6_K through
 * dequant_q6_K_block (dequant.h:291-307).  0 on success, -1 for a type it
 * does not know. */
int ora_dequant_typed_rows(const void *W, int type, float *dst, int rows, int cols);

/* y = W . x, the reference's fp32-activation matvec for the type
 * (q4_matvec / q4_matvec_parallel, mistral_model.h:211-243, 581-644):
 * Q4_K, F16, F32 as dequantised rows dotted in k order (sgemv), Q6_K in the
 * four-lane fma order of q6_K_matvec_f32_neon (dequant.h:365-521), Q4_0 in
 * that of q4_0_matvec_f32 (dequant.h:142-278; the decode layer's W4A8 path
 * for Q4_0 is q4_oracle.h's). */
int ora_typed_matvec(const void *W, int type, const float *x, float *y, int out_dim, int in_dim);

/* The non-Q4_0 branch of q4_matvec_sdot_parallel (mistral_model.h:656-670):
 * x is the Q8_0 blocks' values d * q, then ora_typed_matvec. */
int ora_typed_matvec_q8(const void *W, int type, const OraQ8Block *xq, float *y, int out_dim,
                        int in_dim);

/* tiled_q4_gemm for any type (mistral_ane_prefill.h:1018-1042): Y[S][out_dim]
 * = X[S][in_dim] . dequant(W)^T, fp32 sums in k order; OpenMP over tokens
 * when threads != 1. */
int ora_typed_gemm(const void *W, int type, int out_dim, int in_dim, const float *X, int S,
                   float *Y, int threads);

typedef struct {
    const void *wq, *wk, *wv, *wo, *w1, *w2, *w3; /* [out][in] rows of their type */
    int wq_type, wk_type, wv_type, wo_type, w1_type, w2_type, w3_type;
    const float *rms_att, *rms_ffn;               /* [dim] */
} OraLayerWeightsTyped;

/* blas_prefill_layer (mistral/mistral_ane_prefill.h:1081-1110) with each
 * matrix multiplied by ora_typed_gemm for its own type; otherwise the steps
 * of ora_prefill_layer.  0 on success, -1 for a type it does not know. */
int ora_prefill_layer_typed(const OraLayerWeightsTyped *lw, OraKV *kv, float *X, int layer,
                            int start_pos, int S, int dim, int hidden, int n_heads,
                            int n_kv_heads, float eps, const float *theta_inv, int threads);

/* mistral_layer_decode_parallel (mistral/mistral_model.h:818-899) for one
 * token: x [dim] updated in place, the layer's ring written at pos % max_seq.
 * Composed of the pinned pieces: ora_rmsnorm_batch (S = 1, the same formula
 * as rmsnorm_vec, :202-208), ora_quantize_q8_0, the W4A8 matvec for Q4_0
 * (ora_q4_0_q8_0_matvec; the fused QKV and gate/up dispatches compute the
 * same rows) or ora_typed_matvec_q8 for the other types, ora_decode_step,
 * ora_silu_mul.  0 on success, -1 for a type it does not know. */
int ora_decode_layer_typed(const OraLayerWeightsTyped *lw, OraKV *kv, float *x, int layer,
                           int pos, int dim, int hidden, int n_heads, int n_kv_heads, float eps,
                           const float *theta_inv);

#ifdef __cplusplus
}
#endif

#endif
