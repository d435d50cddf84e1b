/*
 * mia_dropin.h -- drop-in replacement, with the reference's C signatures, for
 * the attention step of the Mistral-7B layer forward.  Needs a compiler with
 * _Float16 (clang, as the reference uses).
 *
 * The reference's path is header-only `static` C (mistral/kv_cache.h,
 * mistral/mistral_model.h, mistral/mistral_ane_prefill.h).  This header keeps
 * the same types (KVCache with the same field order, MistralConfig) and, unless
 * MIA_DROPIN_NO_REFERENCE_NAMES is defined, the same function names as static
 * inline forwards to libmiattn.so.  Differences in behaviour:
 *   - k_cache / v_cache are device memory (the Metal backend re-homes them the
 *     same way, mistral/metal_matvec.h:297-310); kv_k/kv_v/kv_k_at/kv_v_at are
 *     the same pointer arithmetic and return device pointers.
 *   - q, k, out, Q, attn_out, K_buf, V_buf, k_vec, v_vec, theta_inv are host
 *     buffers, as at the reference's call sites; every call is synchronous.
 *   - gqa_attention_neon leaves q unscaled and does not write att (the
 *     reference pre-scales q in place and leaves probabilities in att; no
 *     caller reads either afterwards).
 *   - Errors (no device, unsupported shape, HIP failure) print the reason and
 *     abort(): the reference has no error channel.  mia_dropin_set_abort(0)
 *     makes them return instead, with the message in mia_last_error().
 */
#ifndef MIA_DROPIN_H
#define MIA_DROPIN_H

#include <stddef.h>
#include <stdint.h>

#include "miattn.h"

#ifdef __cplusplus
extern "C" {
#endif

/* mistral/kv_cache.h:10-20, same fields in the same order. */
typedef struct {
    int n_layers;
    int n_kv_heads;
    int head_dim;
    int max_seq;
    int kv_dim;
    _Float16 *k_cache; /* device: [n_layers][max_seq][n_kv_heads][head_dim] */
    _Float16 *v_cache;
    int pos;
    int len;
} KVCache;

/* mistral/gguf_loader.h:51-63, same fields in the same order.  The reference's
 * translation unit includes gguf_loader.h before kv_cache.h
 * (mistral/mistral_infer.m:12-14), so its MistralConfig is already there:
 * gguf_loader.h defines GGUF_MAGIC (gguf_loader.h:15), which suppresses this
 * copy.  A translation unit that includes gguf_loader.h after this header
 * defines MIA_DROPIN_HAVE_MISTRAL_CONFIG first. */
#if !defined(GGUF_MAGIC) && !defined(MIA_DROPIN_HAVE_MISTRAL_CONFIG)
typedef struct {
    int dim;
    int hidden_dim;
    int n_layers;
    int n_heads;
    int n_kv_heads;
    int head_dim;
    int vocab_size;
    int max_seq_len;
    float rope_theta;
    float rms_eps;
    int sliding_window;
} MistralConfig;
#endif

/* mistral/dequant.h:537-541: 36 bytes, fp32 scale then 32 int8. */
typedef struct {
    float d;
    int8_t qs[32];
} mia_block_q8_0;

/* mistral/gguf_loader.h:33 */
#define MIA_GGML_TYPE_Q4_0 2

void mia_dropin_set_abort(int abort_on_error);
int mia_dropin_status(void); /* status of the last drop-in call on this thread */

/* kv_cache.h:22-35 (calloc -> zeroed device memory) */
void mia_dropin_kv_alloc(KVCache *c, int n_layers, int n_kv_heads, int head_dim, int max_seq);
/* kv_cache.h:53-57: host fp16 k_vec/v_vec [kv_dim] -> slot pos % max_seq */
void mia_dropin_kv_write(KVCache *cache, int layer, int pos, const _Float16 *k_vec,
                         const _Float16 *v_vec);
/* kv_cache.h:70-75 */
void mia_dropin_kv_free(KVCache *cache);
/* mistral_model.h:79-122 */
void mia_dropin_apply_rope(float *q, float *k, int pos, const float *theta_inv, int n_heads,
                           int n_kv_heads, int head_dim);
/* mistral_model.h:362-487 */
void mia_dropin_gqa_attention(float *q, float *att, float *out, _Float16 *kcache_base,
                              _Float16 *vcache_base, int n_heads, int heads_per_kv, int hd,
                              int max_seq, int pos);
/* mistral_ane_prefill.h:177-186 */
void mia_dropin_apply_rope_batch(float *Q, float *K, int start_pos, const float *theta_inv,
                                 int n_heads, int n_kv_heads, int head_dim, int S);
/* mistral_ane_prefill.h:189-204 (including the len update) */
void mia_dropin_kv_write_batch(KVCache *kv, int layer, int start_pos, const float *K_buf,
                               const float *V_buf, int kv_dim, int S);
/* mistral_ane_prefill.h:207-275 */
void mia_dropin_attention_batch(const float *Q, float *attn_out, const KVCache *kv, int layer,
                                int start_pos, const MistralConfig *c, int S, float *att_scratch);
/* Steps 4-6 of mistral_model.h:849-863 in one call (RoPE, fp16 cvt, kv_write,
 * len update, attention); q/k/v are the raw projections, not modified. */
void mia_dropin_decode_step(KVCache *kv, int layer, const float *q, const float *k, const float *v,
                            int pos, const float *theta_inv, int n_heads, int n_kv_heads,
                            float *out);
/* The per-layer part of mistral/speculative.h:92-101 for S tokens at once,
 * with the same result as S decode steps (drafts staged, then committed). */
void mia_dropin_verify_step(KVCache *kv, int layer, const float *Q, const float *K, const float *V,
                            int start_pos, int S, const float *theta_inv, int n_heads,
                            int n_kv_heads, float *out);

/* The attention of mistral_layer_prefill_chunk (mistral/mistral_model.h:
 * 908-1075) for one layer: every token's q and k rotated at positions[i], k / v
 * written to slot positions[i] % max_seq (in order: a later token in the same
 * slot wins) with the len update of :952, then each token attends its window
 * over the ring as written (phase 2, :961-1044).  Q, K, V [chunk_size][...]
 * host fp32 raw projections (not modified), positions host int (>= 0),
 * attn_out [chunk_size][n_heads*head_dim] host.  The projections, Wo and the
 * FFN around it stay with the caller. */
void mia_dropin_prefill_chunk_attention(KVCache *kv, int layer, const float *Q, const float *K,
                                        const float *V, const int *positions, int chunk_size,
                                        const float *theta_inv, int n_heads, int n_kv_heads,
                                        float *attn_out);

/* Speculative verify with accept-only commit (mistral/speculative.h:81-105,
 * 242-341): mia_dropin_verify_stage runs one layer's attention for the S
 * verify tokens like mia_dropin_verify_step but leaves the ring untouched,
 * keeping the drafts' K/V in a staging area; once acceptance is known,
 * mia_dropin_verify_commit writes the first n_accepted of every layer and
 * updates len.  Rejected drafts never reach the ring.  One batch at a time;
 * staging a different (start_pos, S) discards an uncommitted batch. */
void mia_dropin_verify_stage(KVCache *kv, int layer, const float *Q, const float *K, const float *V,
                             int start_pos, int S, const float *theta_inv, int n_heads,
                             int n_kv_heads, float *out);
void mia_dropin_verify_commit(KVCache *kv, int start_pos, int n_accepted);

/* W4A8 projections.  Weights W* are device memory holding the Q4_0 blocks as
 * GGUF stores them (the Metal backend re-homes the mmap'd weight file the same
 * way, mistral/metal_matvec.h:185-192, 314); x, x_q8 and y are host buffers. */
/* mistral/dequant.h:545-612 */
void mia_dropin_quantize_q8_0(const float *x, mia_block_q8_0 *out, int n);
/* mistral/mistral_model.h:649-670: Q4_0 on the W4A8 kernel; Q4_K, Q6_K, F16
 * and F32 weights against the Q8_0 values (mia_matvec_q8; other types:
 * MIA_ERR_UNSUPPORTED) */
void mia_dropin_q4_matvec_sdot_parallel(const void *W, uint32_t type, const mia_block_q8_0 *x_q8,
                                        float *y, int out_dim, int in_dim);
/* mistral/mistral_model.h:750-811 */
void mia_dropin_q4_matvec_sdot_parallel_fused_pair(const void *W1, const void *W3,
                                                   const mia_block_q8_0 *x_q8, float *y1,
                                                   float *y3, int out_dim, int in_dim);
/* mistral/mistral_model.h:676-745 */
void mia_dropin_q4_matvec_sdot_parallel_fused_qkv(const void *Wq, const void *Wk, const void *Wv,
                                                  const mia_block_q8_0 *x_q8, float *yq,
                                                  float *yk, float *yv, int dim, int kv_dim,
                                                  int in_dim);

/* The cache saved to / resumed from a file in the snapshot format of
 * mia_kv_snapshot_save (no counterpart in the reference, whose cache lives and
 * dies with the process): k_cache, v_cache, pos and len.  kv_load needs a
 * cache of the same shape from kv_alloc and sets its pos and len.  They
 * return a mia_status (and never abort). */
int mia_dropin_kv_save(const KVCache *c, const char *path);
int mia_dropin_kv_load(KVCache *c, const char *path);

#ifndef MIA_DROPIN_NO_REFERENCE_NAMES
/* Reference names (mistral/kv_cache.h, mistral_model.h, mistral_ane_prefill.h). */
static inline KVCache kv_alloc(int n_layers, int n_kv_heads, int head_dim, int max_seq) {
    KVCache c;
    mia_dropin_kv_alloc(&c, n_layers, n_kv_heads, head_dim, max_seq);
    return c;
}
static inline _Float16 *kv_k_at(const KVCache *cache, int layer, int seq_pos) {
    int t = seq_pos % cache->max_seq;
    return cache->k_cache + (size_t)layer * cache->max_seq * cache->kv_dim +
           (size_t)t * cache->kv_dim;
}
static inline _Float16 *kv_v_at(const KVCache *cache, int layer, int seq_pos) {
    int t = seq_pos % cache->max_seq;
    return cache->v_cache + (size_t)layer * cache->max_seq * cache->kv_dim +
           (size_t)t * cache->kv_dim;
}
static inline void kv_write(KVCache *cache, int layer, int pos, const _Float16 *k_vec,
                            const _Float16 *v_vec) {
    mia_dropin_kv_write(cache, layer, pos, k_vec, v_vec);
}
static inline _Float16 *kv_k(const KVCache *cache, int layer) {
    return cache->k_cache + (size_t)layer * cache->max_seq * cache->kv_dim;
}
static inline _Float16 *kv_v(const KVCache *cache, int layer) {
    return cache->v_cache + (size_t)layer * cache->max_seq * cache->kv_dim;
}
static inline void kv_free(KVCache *cache) { mia_dropin_kv_free(cache); }
static inline void apply_rope(float *q, float *k, int pos, const float *theta_inv, int n_heads,
                              int n_kv_heads, int head_dim) {
    mia_dropin_apply_rope(q, k, pos, theta_inv, n_heads, n_kv_heads, head_dim);
}
static inline void gqa_attention_neon(float *q, float *att, float *out, _Float16 *kcache_base,
                                      _Float16 *vcache_base, int n_heads, int heads_per_kv,
                                      int hd, int max_seq, int pos) {
    mia_dropin_gqa_attention(q, att, out, kcache_base, vcache_base, n_heads, heads_per_kv, hd,
                             max_seq, pos);
}
static inline void apply_rope_batch(float *Q, float *K, int start_pos, const float *theta_inv,
                                    int n_heads, int n_kv_heads, int head_dim, int S) {
    mia_dropin_apply_rope_batch(Q, K, start_pos, theta_inv, n_heads, n_kv_heads, head_dim, S);
}
static inline void kv_write_batch(KVCache *kv, int layer, int start_pos, const float *K_buf,
                                  const float *V_buf, int kv_dim, int S) {
    mia_dropin_kv_write_batch(kv, layer, start_pos, K_buf, V_buf, kv_dim, S);
}
static inline void attention_batch(const float *Q, float *attn_out, const KVCache *kv, int layer,
                                   int start_pos, const MistralConfig *c, int S,
                                   float *att_scratch) {
    mia_dropin_attention_batch(Q, attn_out, kv, layer, start_pos, c, S, att_scratch);
}
#endif /* MIA_DROPIN_NO_REFERENCE_NAMES */

/* The W4A8 names live in mistral/dequant.h, which mistral_model.h includes for
 * every other weight type as well, so they are opt-in: define
 * MIA_DROPIN_Q4_REFERENCE_NAMES in a translation unit that does not include
 * dequant.h.  Elsewhere call the mia_dropin_ forms; mia_block_q8_0 has
 * block_q8_0's layout, so a pointer cast passes the reference's buffers. */
#ifdef MIA_DROPIN_Q4_REFERENCE_NAMES
typedef mia_block_q8_0 block_q8_0;
static inline void quantize_f32_to_q8_0(const float *x, block_q8_0 *out, int n) {
    mia_dropin_quantize_q8_0(x, out, n);
}
static inline void q4_matvec_sdot_parallel(const void *W, uint32_t type, const block_q8_0 *x_q8,
                                           float *y, int out_dim, int in_dim) {
    mia_dropin_q4_matvec_sdot_parallel(W, type, x_q8, y, out_dim, in_dim);
}
static inline void q4_matvec_sdot_parallel_fused_pair(const void *W1, const void *W3,
                                                      const block_q8_0 *x_q8, float *y1,
                                                      float *y3, int out_dim, int in_dim) {
    mia_dropin_q4_matvec_sdot_parallel_fused_pair(W1, W3, x_q8, y1, y3, out_dim, in_dim);
}
static inline void q4_matvec_sdot_parallel_fused_qkv(const void *Wq, const void *Wk,
                                                     const void *Wv, const block_q8_0 *x_q8,
                                                     float *yq, float *yk, float *yv, int dim,
                                                     int kv_dim, int in_dim) {
    mia_dropin_q4_matvec_sdot_parallel_fused_qkv(Wq, Wk, Wv, x_q8, yq, yk, yv, dim, kv_dim,
                                                 in_dim);
}
#endif /* MIA_DROPIN_Q4_REFERENCE_NAMES */

#ifdef __cplusplus
}
#endif
#endif
