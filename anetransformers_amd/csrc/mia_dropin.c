/*
 * mia_dropin.c -- host C side of the drop-in: the reference's attention-step
 * signatures (include/mia_dropin.h) implemented over the libmiattn C ABI.
 * Host buffers are staged through one device buffer owned by this file and
 * its pinned host mirror: a call copies its inputs into the mirror at their
 * device offsets, moves them in one transfer, runs its kernels and brings
 * its outputs back in one transfer, all on the library stream; every call is
 * synchronous, like the reference's.  Not re-entrant (neither is the
 * reference: mistral_model.h shares m->q / m->att across calls).
 */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "../../include/mia_dropin.h"

/* mia_capi.hip, not exported */
int mia_internal_set_error(int code, const char *msg);
int mia_internal_host_alloc(void **p, size_t bytes);
int mia_internal_host_free(void *p);
int mia_internal_copy_async(void *dst, const void *src, size_t bytes, int to_device);

static int g_abort = 1;
static __thread int g_status = 0;
static char *g_dbuf = NULL;  /* device staging */
static char *g_hbuf = NULL;  /* its pinned host mirror, the same size */
static size_t g_dbuf_bytes = 0;

void mia_dropin_set_abort(int abort_on_error) { g_abort = abort_on_error; }
int mia_dropin_status(void) { return g_status; }

static int fail(int rc, const char *what) {
    g_status = rc;
    if (rc && g_abort) {
        fprintf(stderr, "miattn: %s failed (status %d): %s\n", what, rc, mia_last_error());
        abort();
    }
    return rc;
}

#define TRY(what, call)                  \
    do {                                 \
        int rc_ = (call);                \
        if (rc_) {                       \
            fail(rc_, what);             \
            return;                      \
        }                                \
    } while (0)

/* Device staging area of at least `bytes` and its pinned host mirror,
 * carved by the callers (the same offsets in both). */
static int dbuf(size_t bytes) {
    if (bytes <= g_dbuf_bytes) return MIA_OK;
    if (g_dbuf) {
        int rc = mia_free(g_dbuf);
        if (rc) return rc;
    }
    if (g_hbuf) {
        int rc = mia_internal_host_free(g_hbuf);
        if (rc) return rc;
    }
    g_dbuf = NULL;
    g_hbuf = NULL;
    g_dbuf_bytes = 0;
    size_t sz = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
    int rc = mia_malloc((void **)&g_dbuf, sz);
    if (rc) return rc;
    rc = mia_internal_host_alloc((void **)&g_hbuf, sz);
    if (rc) {
        mia_free(g_dbuf);
        g_dbuf = NULL;
        return rc;
    }
    g_dbuf_bytes = sz;
    return MIA_OK;
}

static size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

/* Host input -> the mirror at device offset off (NULL src: nothing). */
static void put(size_t off, const void *src, size_t bytes) {
    if (src && bytes) memcpy(g_hbuf + off, src, bytes);
}
/* The mirror's [0, end) -> the device, one stream-ordered transfer. */
static int push(size_t end) { return mia_internal_copy_async(g_dbuf, g_hbuf, end, 1); }
/* The device's [off, off + bytes) -> the mirror, one transfer, then the
 * stream is synchronised (the kernels before it included). */
static int pull(size_t off, size_t bytes) {
    int rc = mia_internal_copy_async(g_hbuf + off, g_dbuf + off, bytes, 0);
    return rc ? rc : mia_stream_sync(NULL);
}
/* The mirror at device offset off -> a host output. */
static void get(void *dst, size_t off, size_t bytes) {
    if (dst && bytes) memcpy(dst, g_hbuf + off, bytes);
}

void mia_dropin_kv_alloc(KVCache *c, int n_layers, int n_kv_heads, int head_dim, int max_seq) {
    g_status = 0;
    c->n_layers = n_layers;
    c->n_kv_heads = n_kv_heads;
    c->head_dim = head_dim;
    c->max_seq = max_seq;
    c->kv_dim = n_kv_heads * head_dim;
    c->k_cache = NULL;
    c->v_cache = NULL;
    c->pos = 0;
    c->len = 0;
    if (n_layers <= 0 || n_kv_heads <= 0 || head_dim <= 0 || max_seq <= 0) {
        fail(MIA_ERR_INVALID, "kv_alloc (non-positive size)");
        return;
    }
    size_t sz = (size_t)n_layers * max_seq * c->kv_dim * sizeof(_Float16);
    TRY("kv_alloc", mia_malloc((void **)&c->k_cache, sz));
    TRY("kv_alloc", mia_malloc((void **)&c->v_cache, sz));
    TRY("kv_alloc", mia_memset(c->k_cache, 0, sz));
    TRY("kv_alloc", mia_memset(c->v_cache, 0, sz));
}

void mia_dropin_kv_write(KVCache *cache, int layer, int pos, const _Float16 *k_vec,
                         const _Float16 *v_vec) {
    g_status = 0;
    if (layer < 0 || layer >= cache->n_layers || pos < 0) {
        fail(MIA_ERR_INVALID, "kv_write (layer/pos out of range)");
        return;
    }
    size_t sz = (size_t)cache->kv_dim * sizeof(_Float16);
    int t = pos % cache->max_seq;
    size_t off = (size_t)layer * cache->max_seq * cache->kv_dim + (size_t)t * cache->kv_dim;
    TRY("kv_write", mia_memcpy_h2d(cache->k_cache + off, k_vec, sz));
    TRY("kv_write", mia_memcpy_h2d(cache->v_cache + off, v_vec, sz));
}

void mia_dropin_kv_free(KVCache *cache) {
    g_status = 0;
    TRY("kv_free", mia_free(cache->k_cache));
    TRY("kv_free", mia_free(cache->v_cache));
    cache->k_cache = NULL;
    cache->v_cache = NULL;
}

void mia_dropin_apply_rope_batch(float *Q, float *K, int start_pos, const float *theta_inv,
                                 int n_heads, int n_kv_heads, int head_dim, int S) {
    g_status = 0;
    if (S <= 0 || head_dim <= 0) {
        fail(MIA_ERR_INVALID, "apply_rope (bad sizes)");
        return;
    }
    size_t qb = Q ? (size_t)S * n_heads * head_dim * sizeof(float) : 0;
    size_t kb = K ? (size_t)S * n_kv_heads * head_dim * sizeof(float) : 0;
    size_t tb = (size_t)(head_dim / 2) * sizeof(float);
    TRY("apply_rope", dbuf(align256(qb) + align256(kb) + align256(tb)));
    const size_t ko = align256(qb), to = align256(qb) + align256(kb);
    float *dq = Q ? (float *)g_dbuf : NULL;
    float *dk = K ? (float *)(g_dbuf + ko) : NULL;
    float *dt = (float *)(g_dbuf + to);
    put(0, Q, qb);
    put(ko, K, kb);
    put(to, theta_inv, tb);
    TRY("apply_rope", push(to + tb));
    TRY("apply_rope", mia_rope_f32(dq, dk, S, start_pos, dt, n_heads, n_kv_heads, head_dim, NULL));
    TRY("apply_rope", pull(0, to));
    get(Q, 0, qb);
    get(K, ko, kb);
}

void mia_dropin_apply_rope(float *q, float *k, int pos, const float *theta_inv, int n_heads,
                           int n_kv_heads, int head_dim) {
    mia_dropin_apply_rope_batch(q, k, pos, theta_inv, n_heads, n_kv_heads, head_dim, 1);
}

void mia_dropin_gqa_attention(float *q, float *att, float *out, _Float16 *kcache_base,
                              _Float16 *vcache_base, int n_heads, int heads_per_kv, int hd,
                              int max_seq, int pos) {
    (void)att;
    g_status = 0;
    if (n_heads <= 0 || hd <= 0) {
        fail(MIA_ERR_INVALID, "gqa_attention (bad sizes)");
        return;
    }
    size_t nb = (size_t)n_heads * hd * sizeof(float);
    TRY("gqa_attention", dbuf(2 * align256(nb)));
    float *dq = (float *)g_dbuf;
    float *dout = (float *)(g_dbuf + align256(nb));
    put(0, q, nb);
    TRY("gqa_attention", push(nb));
    TRY("gqa_attention", mia_gqa_attention(dq, dout, (const uint16_t *)kcache_base,
                                           (const uint16_t *)vcache_base, n_heads, heads_per_kv, hd,
                                           max_seq, pos, NULL));
    TRY("gqa_attention", pull(align256(nb), nb));
    get(out, align256(nb), nb);
}

void mia_dropin_kv_write_batch(KVCache *kv, int layer, int start_pos, const float *K_buf,
                               const float *V_buf, int kv_dim, int S) {
    g_status = 0;
    if (layer < 0 || layer >= kv->n_layers || kv_dim != kv->kv_dim || S <= 0) {
        fail(MIA_ERR_INVALID, "kv_write_batch (bad layer/kv_dim/S)");
        return;
    }
    size_t nb = (size_t)S * kv_dim * sizeof(float);
    TRY("kv_write_batch", dbuf(2 * align256(nb)));
    float *dk = (float *)g_dbuf;
    float *dv = (float *)(g_dbuf + align256(nb));
    put(0, K_buf, nb);
    put(align256(nb), V_buf, nb);
    TRY("kv_write_batch", push(align256(nb) + nb));
    size_t lay = (size_t)layer * kv->max_seq * kv->kv_dim;
    TRY("kv_write_batch", mia_kv_write_f32((uint16_t *)(kv->k_cache + lay),
                                           (uint16_t *)(kv->v_cache + lay), dk, dv, S, start_pos,
                                           kv->max_seq, kv_dim, NULL));
    TRY("kv_write_batch", mia_stream_sync(NULL));
    /* mistral_ane_prefill.h:201-203 */
    int end_pos = start_pos + S;
    if (end_pos > kv->len && end_pos <= kv->max_seq)
        kv->len = end_pos;
    else if (end_pos > kv->max_seq)
        kv->len = kv->max_seq;
}

void mia_dropin_attention_batch(const float *Q, float *attn_out, const KVCache *kv, int layer,
                                int start_pos, const MistralConfig *c, int S, float *att_scratch) {
    (void)att_scratch;
    g_status = 0;
    if (layer < 0 || layer >= kv->n_layers || S <= 0 || c->dim != c->n_heads * c->head_dim) {
        fail(MIA_ERR_INVALID, "attention_batch (bad layer/S/dim)");
        return;
    }
    size_t nb = (size_t)S * c->dim * sizeof(float);
    TRY("attention_batch", dbuf(2 * align256(nb)));
    float *dq = (float *)g_dbuf;
    float *dout = (float *)(g_dbuf + align256(nb));
    put(0, Q, nb);
    TRY("attention_batch", push(nb));
    size_t lay = (size_t)layer * kv->max_seq * kv->kv_dim;
    TRY("attention_batch",
        mia_attention_batch(dq, dout, (const uint16_t *)(kv->k_cache + lay),
                            (const uint16_t *)(kv->v_cache + lay), c->n_heads, c->n_kv_heads,
                            c->head_dim, kv->max_seq, start_pos, S, NULL));
    TRY("attention_batch", pull(align256(nb), nb));
    get(attn_out, align256(nb), nb);
}

void mia_dropin_prefill_chunk_attention(KVCache *kv, int layer, const float *Q, const float *K,
                                        const float *V, const int *positions, int chunk_size,
                                        const float *theta_inv, int n_heads, int n_kv_heads,
                                        float *attn_out) {
    const char *what = "prefill_chunk_attention";
    g_status = 0;
    if (layer < 0 || layer >= kv->n_layers || chunk_size <= 0 || n_heads <= 0 ||
        n_kv_heads <= 0 || n_kv_heads * kv->head_dim != kv->kv_dim) {
        fail(MIA_ERR_INVALID, what);
        return;
    }
    for (int i = 0; i < chunk_size; i++)
        if (positions[i] < 0) {
            fail(MIA_ERR_INVALID, "prefill_chunk_attention (negative position)");
            return;
        }
    int hd = kv->head_dim;
    size_t qb = (size_t)chunk_size * n_heads * hd * sizeof(float);
    size_t kb = (size_t)chunk_size * kv->kv_dim * sizeof(float);
    size_t tb = (size_t)(hd / 2) * sizeof(float);
    size_t pb = (size_t)chunk_size * sizeof(int);
    size_t a = align256(qb), b = align256(kb), t = align256(tb), pp = align256(pb);
    TRY(what, dbuf(2 * a + 2 * b + t + pp));
    float *dq = (float *)g_dbuf;
    float *dk = (float *)(g_dbuf + a);
    float *dv = (float *)(g_dbuf + a + b);
    float *dt = (float *)(g_dbuf + a + 2 * b);
    int *dp = (int *)(g_dbuf + a + 2 * b + t);
    float *dout = (float *)(g_dbuf + a + 2 * b + t + pp);
    put(0, Q, qb);
    put(a, K, kb);
    put(a + b, V, kb);
    put(a + 2 * b, theta_inv, tb);
    put(a + 2 * b + t, positions, pb);
    TRY(what, push(a + 2 * b + t + pb));
    size_t lay = (size_t)layer * kv->max_seq * kv->kv_dim;
    TRY(what, mia_attention_chunk(dq, dk, dv, dp, dt, (uint16_t *)(kv->k_cache + lay),
                                  (uint16_t *)(kv->v_cache + lay), dout, n_heads, n_kv_heads, hd,
                                  kv->max_seq, chunk_size, NULL));
    TRY(what, pull(a + 2 * b + t + pp, qb));
    get(attn_out, a + 2 * b + t + pp, qb);
    /* mistral_model.h:952, per token */
    for (int i = 0; i < chunk_size; i++)
        if (kv->len < kv->max_seq && positions[i] + 1 > kv->len) kv->len = positions[i] + 1;
}

/* Staged verify rows: [n_layers][S][kv_dim] fp16 K, then the same for V, for
 * one batch of drafts (start_pos, S) at a time. */
static uint16_t *g_stage = NULL;
static size_t g_stage_bytes = 0;
static int g_stage_start = -1, g_stage_S = 0, g_stage_layers = 0;
static unsigned char *g_stage_done = NULL; /* per layer: staged for this batch */

static int stage_for(KVCache *kv, int start_pos, int S) {
    size_t need = 2 * (size_t)kv->n_layers * S * kv->kv_dim * sizeof(uint16_t);
    if (g_stage_start != start_pos || g_stage_S != S || g_stage_layers != kv->n_layers) {
        if (need > g_stage_bytes) {
            if (g_stage) {
                int rc = mia_free(g_stage);
                if (rc) return rc;
            }
            g_stage = NULL;
            g_stage_bytes = 0;
            int rc = mia_malloc((void **)&g_stage, need);
            if (rc) return rc;
            g_stage_bytes = need;
        }
        unsigned char *done = (unsigned char *)realloc(g_stage_done, (size_t)kv->n_layers);
        if (!done) return mia_internal_set_error(MIA_ERR_INVALID, "out of host memory");
        g_stage_done = done;
        memset(g_stage_done, 0, (size_t)kv->n_layers);
        g_stage_start = start_pos;
        g_stage_S = S;
        g_stage_layers = kv->n_layers;
    }
    return MIA_OK;
}

static void step_common(const char *what, KVCache *kv, int layer, const float *Q, const float *K,
                        const float *V, int start_pos, int S, const float *theta_inv, int n_heads,
                        int n_kv_heads, float *out, int staged) {
    g_status = 0;
    if (layer < 0 || layer >= kv->n_layers || S <= 0 || n_heads <= 0 || n_kv_heads <= 0 ||
        n_kv_heads * kv->head_dim != kv->kv_dim) {
        fail(MIA_ERR_INVALID, what);
        return;
    }
    if (staged) TRY(what, stage_for(kv, start_pos, S));
    int hd = kv->head_dim;
    size_t qb = (size_t)S * n_heads * hd * sizeof(float);
    size_t kb = (size_t)S * kv->kv_dim * sizeof(float);
    size_t tb = (size_t)(hd / 2) * sizeof(float);
    size_t a = align256(qb), b = align256(kb), t = align256(tb);
    TRY(what, dbuf(2 * a + 2 * b + t));
    float *dq = (float *)g_dbuf;
    float *dk = (float *)(g_dbuf + a);
    float *dv = (float *)(g_dbuf + a + b);
    float *dt = (float *)(g_dbuf + a + 2 * b);
    float *dout = (float *)(g_dbuf + a + 2 * b + t);
    put(0, Q, qb);
    put(a, K, kb);
    put(a + b, V, kb);
    put(a + 2 * b, theta_inv, tb);
    TRY(what, push(a + 2 * b + tb));
    size_t lay = (size_t)layer * kv->max_seq * kv->kv_dim;
    if (staged) {
        size_t rows = (size_t)S * kv->kv_dim;
        uint16_t *ks = g_stage + (size_t)layer * rows;
        uint16_t *vs = g_stage + (size_t)kv->n_layers * rows + (size_t)layer * rows;
        TRY(what, mia_attention_step_staged(dq, dk, dv, dt, (uint16_t *)(kv->k_cache + lay),
                                            (uint16_t *)(kv->v_cache + lay), ks, vs, dout,
                                            n_heads, n_kv_heads, hd, kv->max_seq, start_pos, S,
                                            NULL));
    } else {
        TRY(what, mia_attention_step(dq, dk, dv, dt, (uint16_t *)(kv->k_cache + lay),
                                     (uint16_t *)(kv->v_cache + lay), dout, n_heads, n_kv_heads,
                                     hd, kv->max_seq, start_pos, S, NULL));
    }
    TRY(what, pull(a + 2 * b + t, qb));
    get(out, a + 2 * b + t, qb);
    if (staged) {
        g_stage_done[layer] = 1;
        return; /* the ring and len change at commit */
    }
    /* mistral_model.h:858, once per token as the sequential steps do */
    for (int i = 0; i < S; i++) {
        int pos = start_pos + i;
        if (kv->len < kv->max_seq && pos + 1 > kv->len) kv->len = pos + 1;
    }
}

void mia_dropin_decode_step(KVCache *kv, int layer, const float *q, const float *k, const float *v,
                            int pos, const float *theta_inv, int n_heads, int n_kv_heads,
                            float *out) {
    step_common("decode_step", kv, layer, q, k, v, pos, 1, theta_inv, n_heads, n_kv_heads, out, 0);
}

void mia_dropin_verify_step(KVCache *kv, int layer, const float *Q, const float *K, const float *V,
                            int start_pos, int S, const float *theta_inv, int n_heads,
                            int n_kv_heads, float *out) {
    step_common("verify_step", kv, layer, Q, K, V, start_pos, S, theta_inv, n_heads, n_kv_heads,
                out, 0);
}

void mia_dropin_quantize_q8_0(const float *x, mia_block_q8_0 *out, int n) {
    g_status = 0;
    if (n <= 0 || n % 32) {
        fail(MIA_ERR_INVALID, "quantize_f32_to_q8_0 (n not a positive multiple of 32)");
        return;
    }
    size_t xb = (size_t)n * sizeof(float);
    size_t qb = (size_t)(n / 32) * sizeof(mia_block_q8_0);
    TRY("quantize_f32_to_q8_0", dbuf(align256(xb) + align256(qb)));
    float *dx = (float *)g_dbuf;
    void *dq = g_dbuf + align256(xb);
    put(0, x, xb);
    TRY("quantize_f32_to_q8_0", push(xb));
    TRY("quantize_f32_to_q8_0", mia_quantize_q8_0(dx, dq, n, NULL));
    TRY("quantize_f32_to_q8_0", pull(align256(xb), qb));
    get(out, align256(xb), qb);
}

void mia_dropin_q4_matvec_sdot_parallel_fused_qkv(const void *Wq, const void *Wk, const void *Wv,
                                                  const mia_block_q8_0 *x_q8, float *yq,
                                                  float *yk, float *yv, int dim, int kv_dim,
                                                  int in_dim) {
    const char *what = "q4_matvec_sdot_parallel";
    g_status = 0;
    if (dim <= 0 || kv_dim < 0 || in_dim <= 0 || in_dim % 32) {
        fail(MIA_ERR_INVALID, "q4_matvec (bad sizes)");
        return;
    }
    size_t xb = (size_t)(in_dim / 32) * sizeof(mia_block_q8_0);
    size_t qb = (size_t)dim * sizeof(float), kb = (size_t)kv_dim * sizeof(float);
    TRY(what, dbuf(align256(xb) + align256(qb) + 2 * align256(kb)));
    void *dx = g_dbuf;
    float *dyq = (float *)(g_dbuf + align256(xb));
    float *dyk = kv_dim ? (float *)(g_dbuf + align256(xb) + align256(qb)) : NULL;
    float *dyv = kv_dim ? (float *)(g_dbuf + align256(xb) + align256(qb) + align256(kb)) : NULL;
    put(0, x_q8, xb);
    TRY(what, push(xb));
    TRY(what, mia_q4_0_matvec_qkv(Wq, Wk, Wv, dx, dyq, dyk, dyv, dim, kv_dim, in_dim, NULL));
    const size_t yo = align256(xb);
    TRY(what, pull(yo, kv_dim ? align256(qb) + align256(kb) + kb : qb));
    get(yq, yo, qb);
    if (kv_dim) {
        get(yk, yo + align256(qb), kb);
        get(yv, yo + align256(qb) + align256(kb), kb);
    }
}

void mia_dropin_q4_matvec_sdot_parallel_fused_pair(const void *W1, const void *W3,
                                                   const mia_block_q8_0 *x_q8, float *y1,
                                                   float *y3, int out_dim, int in_dim) {
    const char *what = "q4_matvec_sdot_parallel_fused_pair";
    g_status = 0;
    if (out_dim <= 0 || in_dim <= 0 || in_dim % 32) {
        fail(MIA_ERR_INVALID, "q4_matvec (bad sizes)");
        return;
    }
    size_t xb = (size_t)(in_dim / 32) * sizeof(mia_block_q8_0);
    size_t yb = (size_t)out_dim * sizeof(float);
    TRY(what, dbuf(align256(xb) + 2 * align256(yb)));
    void *dx = g_dbuf;
    float *dy1 = (float *)(g_dbuf + align256(xb));
    float *dy3 = (float *)(g_dbuf + align256(xb) + align256(yb));
    put(0, x_q8, xb);
    TRY(what, push(xb));
    TRY(what, mia_q4_0_matvec_pair(W1, W3, dx, dy1, dy3, out_dim, in_dim, NULL));
    TRY(what, pull(align256(xb), align256(yb) + yb));
    get(y1, align256(xb), yb);
    get(y3, align256(xb) + align256(yb), yb);
}

void mia_dropin_q4_matvec_sdot_parallel(const void *W, uint32_t type, const mia_block_q8_0 *x_q8,
                                        float *y, int out_dim, int in_dim) {
    const char *what = "q4_matvec_sdot_parallel";
    g_status = 0;
    if (type == MIA_GGML_TYPE_Q4_0) {
        mia_dropin_q4_matvec_sdot_parallel_fused_qkv(W, NULL, NULL, x_q8, y, NULL, NULL, out_dim,
                                                     0, in_dim);
        return;
    }
    /* every other type: the Q8_0 values d * q against the type's weights
     * (mistral_model.h:656-670) */
    if (out_dim <= 0 || in_dim <= 0 || in_dim % 32) {
        fail(MIA_ERR_INVALID, "q4_matvec (bad sizes)");
        return;
    }
    size_t xb = (size_t)(in_dim / 32) * sizeof(mia_block_q8_0);
    size_t yb = (size_t)out_dim * sizeof(float);
    TRY(what, dbuf(align256(xb) + align256(yb)));
    void *dx = g_dbuf;
    float *dy = (float *)(g_dbuf + align256(xb));
    put(0, x_q8, xb);
    TRY(what, push(xb));
    TRY(what, mia_matvec_q8(W, (int)type, dx, dy, out_dim, in_dim, NULL));
    TRY(what, pull(align256(xb), yb));
    get(y, align256(xb), yb);
}

void mia_dropin_verify_stage(KVCache *kv, int layer, const float *Q, const float *K, const float *V,
                             int start_pos, int S, const float *theta_inv, int n_heads,
                             int n_kv_heads, float *out) {
    step_common("verify_stage", kv, layer, Q, K, V, start_pos, S, theta_inv, n_heads, n_kv_heads,
                out, 1);
}

void mia_dropin_verify_commit(KVCache *kv, int start_pos, int n_accepted) {
    const char *what = "verify_commit";
    g_status = 0;
    if (g_stage_start != start_pos || g_stage_layers != kv->n_layers || n_accepted < 0 ||
        n_accepted > g_stage_S) {
        fail(MIA_ERR_INVALID, "verify_commit (no staged batch at this start_pos, or n_accepted "
                              "above its size)");
        return;
    }
    for (int l = 0; l < kv->n_layers; l++) {
        if (!g_stage_done[l]) {
            fail(MIA_ERR_INVALID, "verify_commit (a layer of the batch was not staged)");
            return;
        }
    }
    size_t rows = (size_t)g_stage_S * kv->kv_dim;
    TRY(what, mia_commit_staged((uint16_t *)kv->k_cache, (uint16_t *)kv->v_cache, g_stage,
                                g_stage + (size_t)kv->n_layers * rows, kv->n_layers, g_stage_S,
                                n_accepted, start_pos, kv->max_seq, kv->kv_dim, NULL));
    TRY(what, mia_stream_sync(NULL));
    /* mistral_model.h:858, once per committed token */
    for (int i = 0; i < n_accepted; i++) {
        int pos = start_pos + i;
        if (kv->len < kv->max_seq && pos + 1 > kv->len) kv->len = pos + 1;
    }
    g_stage_start = -1; /* the batch is spent */
}
