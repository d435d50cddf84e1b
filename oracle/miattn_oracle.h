/*
 * miattn_oracle.h -- CPU oracle for the Mistral-7B GQA attention hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a portable scalar-C restatement of the
 * reference's CPU attention (NEON -> scalar, Accelerate -> libm / plain loops).
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it, and only as the checker or the timed CPU baseline.  The product
 * library (libmiattn.so) never links, loads or calls it.
 *
 * fp16 storage is uint16_t (IEEE binary16 bit patterns), so gcc builds it.
 *
 * Pinning status per function (what checks it in tests/test_oracle.py):
 *   ora_f32_to_f16 / ora_f16_to_f32   exhaustive vs numpy float16 (RNE)    pinned
 *   ora_precompute_rope_theta         closed form in float64               pinned
 *   ora_apply_rope                    pos=0 identity, norm preservation,
 *                                     float64 rotation on the fp32 angle    pinned
 *   ora_softmax_vec                   uniform / dominant known answers,
 *                                     float64 softmax                       pinned
 *   ora_kv_*                          slot = pos % max_seq closed form      pinned
 *   ora_gqa_attention                 float64 brute force, L=1 -> V row,
 *                                     equal keys -> mean(V), GQA broadcast  pinned
 *   ora_attention_batch               == S sequential ora_gqa_attention
 *                                     steps (unwrapped), textbook causal    pinned
 *   ora_ref_gqa_attention             float64 brute force                   pinned
 *   ora_decode_step / ora_verify_steps  compositions of the above           pinned
 *   ora_prefill_chunk_attention       == sequential steps (unwrapped, in
 *                                     order), float64 brute force over the
 *                                     final ring for any positions          pinned
 * The transcendental boundary (Accelerate vvsincosf / vvexpf, replaced here by
 * libm sinf/cosf/expf) is parity-unpinned: no reference test fixes those
 * outputs; ulp-level differences are inside the attention tolerance.
 */
#ifndef MIATTN_ORACLE_H
#define MIATTN_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* fp32 <-> IEEE binary16, round-to-nearest-even (vcvt_f16_f32 with the
 * default FPCR, as used by mistral/mistral_model.h:160-169). */
uint16_t ora_f32_to_f16(float f);
float ora_f16_to_f32(uint16_t h);
void ora_cvt_f32_to_f16(const float *src, uint16_t *dst, int n);
void ora_cvt_f16_to_f32(const uint16_t *src, float *dst, size_t n);

/* mistral/mistral_model.h:69-74 */
void ora_precompute_rope_theta(float rope_theta, int head_dim, float *theta_inv);

/* mistral/mistral_model.h:79-122 (in place, adjacent pairs) */
void ora_apply_rope(float *q, float *k, int pos, const float *theta_inv,
                    int n_heads, int n_kv_heads, int head_dim);

/* mistral/mistral_ane_prefill.h:177-186 */
void ora_apply_rope_batch(float *Q, float *K, int start_pos, const float *theta_inv,
                          int n_heads, int n_kv_heads, int head_dim, int S);

/* mistral/mistral_model.h:245-256 */
void ora_softmax_vec(float *x, int n);

/* mistral/kv_cache.h:10-20, same field order. */
typedef struct {
    int n_layers;
    int n_kv_heads;
    int head_dim;
    int max_seq;
    int kv_dim;
    uint16_t *k_cache; /* [n_layers][max_seq][n_kv_heads][head_dim] */
    uint16_t *v_cache;
    int pos;
    int len;
} OraKV;

int ora_kv_alloc(OraKV *c, int n_layers, int n_kv_heads, int head_dim, int max_seq); /* kv_cache.h:22-35 */
uint16_t *ora_kv_k_at(const OraKV *c, int layer, int seq_pos);                       /* :38-42 */
uint16_t *ora_kv_v_at(const OraKV *c, int layer, int seq_pos);                       /* :45-49 */
void ora_kv_write(OraKV *c, int layer, int pos, const uint16_t *k_vec, const uint16_t *v_vec); /* :53-57 */
uint16_t *ora_kv_k(const OraKV *c, int layer);                                       /* :61-63 */
uint16_t *ora_kv_v(const OraKV *c, int layer);                                       /* :66-68 */
void ora_kv_free(OraKV *c);                                                          /* :70-75 */

/* mistral/mistral_model.h:362-487.  q is pre-scaled in place (as the
 * reference does); att [n_heads * max_seq] is left holding probabilities. */
void ora_gqa_attention(float *q, float *att, float *out,
                       const uint16_t *kcache_base, const uint16_t *vcache_base,
                       int n_heads, int heads_per_kv, int hd, int max_seq, int pos);

/* mistral/mistral_ane_prefill.h:189-204 */
void ora_kv_write_batch(OraKV *kv, int layer, int start_pos,
                        const float *K_buf, const float *V_buf, int kv_dim, int S);

/* mistral/mistral_ane_prefill.h:207-275 (att_scratch [n_heads * max_seq]). */
void ora_attention_batch(const float *Q, float *attn_out, const OraKV *kv, int layer,
                         int start_pos, int n_heads, int n_kv_heads, int head_dim,
                         int S, float *att_scratch);

/* Steps 4-6 of mistral/mistral_model.h:849-863: RoPE(q, k) at pos, fp16 cvt,
 * kv_write at pos % max_seq, len update, gqa_attention.  q and k are rotated in
 * place (q also pre-scaled); v is read only.  out [n_heads * hd]. */
void ora_decode_step(OraKV *kv, int layer, float *q, float *k, const float *v, int pos,
                     const float *theta_inv, int n_heads, int n_kv_heads, float *att,
                     float *out);

/* mistral/speculative.h:92-101 semantics for one layer: S sequential decode
 * steps at start_pos + t (write token t, then attend).  Q [S][n_heads*hd],
 * K/V [S][kv_dim] raw (unrotated) fp32; Q and K are overwritten. */
void ora_verify_steps(OraKV *kv, int layer, float *Q, float *K, const float *V, int start_pos,
                      int S, const float *theta_inv, int n_heads, int n_kv_heads, float *att,
                      float *out);

/* mistral/mistral_model.h:908-1075, the attention of the chunked prefill
 * layer: phase 1 (:935-955) rotates q and k of every token at positions[t],
 * writes fp16 k / v to slot positions[t] % max_seq in token order (a later
 * token in the same slot wins) and updates len; phase 2 (:961-1044) attends
 * every token over the ring as phase 1 left it, at pos = positions[t].  Q, K
 * [S][...] raw fp32, overwritten (Q ends rotated and pre-scaled, as Q_all).
 * The projections, Wo and the FFN of that function are not part of this. */
void ora_prefill_chunk_attention(OraKV *kv, int layer, float *Q, float *K, const float *V,
                                 const int *positions, int S, const float *theta_inv,
                                 int n_heads, int n_kv_heads, float *att, float *out);

/* tests/test_cpu_ref.h:113-147: textbook causal GQA over contiguous
 * [S][n_kv][hd] K/V starting at position 0. */
void ora_ref_gqa_attention(float *out, const float *q, const float *k, const float *v, int S,
                           int n_heads, int n_kv_heads, int head_dim);

/* CPU baseline driver (timing only): decode attention for n_layers
 * independent layer caches, each layer = one ora_gqa_attention call over the
 * ring as it stands.  Q [n_layers][n_heads*hd] (copied, not mutated), out
 * [n_layers][n_heads*hd].  Parallelised with OpenMP over (layer, kv head)
 * when built with -fopenmp; n_threads <= 0 keeps the OpenMP default. */
void ora_decode_layers(const float *Q, float *out, const uint16_t *k_cache,
                       const uint16_t *v_cache, int n_layers, int n_heads, int heads_per_kv,
                       int hd, int max_seq, int pos, int n_threads);

/* Same, for attention_batch over n_layers layers (prefill chunk). */
void ora_attention_batch_layers(const float *Q, float *out, const uint16_t *k_cache,
                                const uint16_t *v_cache, int n_layers, int n_heads,
                                int n_kv_heads, int hd, int max_seq, int start_pos, int S,
                                int n_threads);

int ora_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
