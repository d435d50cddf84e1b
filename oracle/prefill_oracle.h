/*
 * prefill_oracle.h -- CPU oracle for the GPU prefill layer: RMSNorm, the Q4_0
 * GEMM on fp32 activations, SwiGLU and the layer that chains them with the
 * attention step (mistral/mistral_ane_prefill.h:1081-1110).
 *
 * TEST INFRASTRUCTURE ONLY, like miattn_oracle.h: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Pinning status (tests/test_oracle_prefill.py):
 *   ora_rmsnorm_batch       known answers (constant and zero rows) and a
 *                           float64 restatement of the formula        pinned
 *   ora_dequant_q4_0_rows   equal to the float64 dequantisation pinned by
 *                           the Q4 tests (exact in fp32)              pinned
 *   ora_q4_0_gemm           float64 matmul of dequantised weights     pinned
 *   ora_silu_mul            known answers (0, large +-) and float64   pinned
 *   ora_prefill_layer       a float64 numpy layer (RMSNorm, GEMMs, RoPE,
 *                           causal attention over the ring, SwiGLU)   pinned
 * The order of the GEMM's and the dot product's fp32 sums (BLAS, vDSP) is not
 * fixed by the reference; exp comes from libm here and vvexpf there: parity
 * unpinned at the ulp level, inside the tolerance.
 */
#ifndef PREFILL_ORACLE_H
#define PREFILL_ORACLE_H

#include "miattn_oracle.h"

#ifdef __cplusplus
extern "C" {
#endif

/* mistral/mistral_ane_prefill.h:163-175 */
void ora_rmsnorm_batch(float *out, const float *in, const float *w, int dim, int S, float eps);

/* mistral/mistral_ane_prefill.h:907-943 (Q4_0 branch): rows x cols fp32 */
void ora_dequant_q4_0_rows(const void *W, float *dst, int rows, int cols);

/* mistral/mistral_ane_prefill.h:999-1042: Y[S][out_dim] = X[S][in_dim] .
 * dequant(W)^T, fp32 sums in k order; OpenMP over tokens when threads != 1. */
void ora_q4_0_gemm(const void *W, int out_dim, int in_dim, const float *X, int S, float *Y,
                   int threads);

/* mistral/mistral_model.h:174-199: gate[i] = gate[i] * (1 / (1 + exp(-gate[i]))) * up[i] */
void ora_silu_mul(float *gate, const float *up, int n);

typedef struct {
    const void *wq, *wk, *wv, *wo, *w1, *w2, *w3; /* Q4_0 [out][in] */
    const float *rms_att, *rms_ffn;              /* [dim] */
} OraLayerWeights;

/* mistral/mistral_ane_prefill.h:1081-1110: X [S][dim] updated in place, the
 * layer's ring written at start_pos..start_pos+S-1. */
void ora_prefill_layer(const OraLayerWeights *lw, OraKV *kv, float *X, int layer, int start_pos,
                       int S, int dim, int hidden, int n_heads, int n_kv_heads, float eps,
                       const float *theta_inv, int threads);

#ifdef __cplusplus
}
#endif

#endif
