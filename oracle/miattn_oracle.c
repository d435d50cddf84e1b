/*
 * miattn_oracle.c -- CPU oracle (test infrastructure only; see the header).
 *
 * Scalar restatement of the reference's CPU attention path.  Each function
 * cites the reference file:line it follows.  Substitutions:
 *   NEON fp32 lanes            -> scalar loops keeping the lane/accumulator order
 *   vfmaq_f32 / vfmsq_f32      -> fmaf (fused, as the NEON instructions are)
 *   vcvt_f16_f32 / vcvt_f32_f16 -> ora_f32_to_f16 / ora_f16_to_f32 (RNE)
 *   vDSP_vsmul + vvsincosf     -> fp32 multiply + libm sinf / cosf
 *   vvexpf                     -> libm expf
 *   vDSP_maxv / vsadd / sve / vsmul -> sequential loops
 * Build without -ffast-math and with -ffp-contract=off for parity; the timing
 * build adds the reference's -ffast-math (mistral/Makefile:2) and ORA_SIMD.
 */
#include "miattn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif
#ifdef __F16C__
#include <immintrin.h>
#endif
/* ORA_SIMD (timing build only): AVX2 + F16C versions of the dot and
 * weighted-V loops, the x86 counterpart of the reference's NEON loops.  The
 * parity build keeps the scalar code that follows the NEON lane order. */
#if defined(ORA_SIMD) && defined(__AVX2__) && defined(__F16C__) && defined(__FMA__)
#define ORA_USE_AVX2 1
static inline float hsum256(__m256 v) {
    __m128 lo = _mm256_castps256_ps128(v), hi = _mm256_extractf128_ps(v, 1);
    lo = _mm_add_ps(lo, hi);
    lo = _mm_hadd_ps(lo, lo);
    lo = _mm_hadd_ps(lo, lo);
    return _mm_cvtss_f32(lo);
}
static inline float dot_avx2(const float *q, const uint16_t *k, int hd) {
    __m256 a0 = _mm256_setzero_ps(), a1 = _mm256_setzero_ps();
    for (int d = 0; d < hd; d += 16) {
        __m256 k0 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(k + d)));
        __m256 k1 = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(k + d + 8)));
        a0 = _mm256_fmadd_ps(_mm256_loadu_ps(q + d), k0, a0);
        a1 = _mm256_fmadd_ps(_mm256_loadu_ps(q + d + 8), k1, a1);
    }
    return hsum256(_mm256_add_ps(a0, a1));
}
static inline void axpy_avx2(float a, const uint16_t *v, float *o, int hd) {
    __m256 av = _mm256_set1_ps(a);
    for (int d = 0; d < hd; d += 8) {
        __m256 vv = _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)(v + d)));
        _mm256_storeu_ps(o + d, _mm256_fmadd_ps(av, vv, _mm256_loadu_ps(o + d)));
    }
}
#endif

/* ---------------------------------------------------------------- fp16 -- */

uint16_t ora_f32_to_f16(float f) {
#ifdef __F16C__
    /* vcvtps2ph with round-to-nearest-even: same bits as the portable path */
    return (uint16_t)_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
#endif
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t ax = x & 0x7fffffffu;
    if (ax >= 0x7f800000u) { /* inf / nan */
        if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
        return (uint16_t)(sign | 0x7c00u);
    }
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* >= 65520 -> inf */
    if (ax >= 0x38800000u) {                                  /* normal half */
        uint32_t r = ax + 0xfffu + ((ax >> 13) & 1u);         /* RNE at bit 13 */
        r -= 0x38000000u;                                     /* rebias 127 -> 15 */
        return (uint16_t)(sign | (r >> 13));
    }
    if (ax <= 0x33000000u) return (uint16_t)sign; /* <= 2^-25 -> +-0 (tie to even) */
    /* half subnormal: m = round(|f| / 2^-24), RNE */
    uint32_t e = ax >> 23;
    uint32_t mant = (ax & 0x7fffffu) | 0x800000u;
    uint32_t shift = 126u - e; /* 14..24 */
    uint32_t m = mant >> shift;
    uint32_t rem = mant & ((1u << shift) - 1u);
    uint32_t half = 1u << (shift - 1u);
    if (rem > half || (rem == half && (m & 1u))) m++;
    return (uint16_t)(sign | m);
}

float ora_f16_to_f32(uint16_t h) {
#ifdef __F16C__
    return _cvtsh_ss(h); /* exact */
#endif
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t e = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t m = (uint32_t)h & 0x3ffu;
    uint32_t bits;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
        return sign ? -v : v;
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* mistral/mistral_model.h:160-169 (cvt_f32_to_f16_neon); identical to
 * mistral/mistral_ane_prefill.h:63-74 (cvt_f32_to_f16). */
void ora_cvt_f32_to_f16(const float *src, uint16_t *dst, int n) {
    for (int i = 0; i < n; i++) dst[i] = ora_f32_to_f16(src[i]);
}

void ora_cvt_f16_to_f32(const uint16_t *src, float *dst, size_t n) {
    for (size_t i = 0; i < n; i++) dst[i] = ora_f16_to_f32(src[i]);
}

/* ---------------------------------------------------------------- RoPE -- */

/* mistral/mistral_model.h:69-74 */
void ora_precompute_rope_theta(float rope_theta, int head_dim, float *theta_inv) {
    int hd2 = head_dim / 2;
    for (int i = 0; i < hd2; i++)
        theta_inv[i] = 1.0f / powf(rope_theta, (2.0f * i) / head_dim);
}

static void rope_rotate(float *x, int n_vec, int head_dim, const float *cos_tab,
                        const float *sin_tab) {
    int hd2 = head_dim / 2;
    for (int h = 0; h < n_vec; h++) {
        float *xh = x + (size_t)h * head_dim;
        for (int i = 0; i < hd2; i++) {
            float c = cos_tab[i], s = sin_tab[i];
            float e = xh[2 * i], o = xh[2 * i + 1];
            /* :100-105: even*cos - odd*sin (vfmsq over vmulq), odd*cos + even*sin */
            float ec = e * c;
            float oc = o * c;
            xh[2 * i] = fmaf(-o, s, ec);
            xh[2 * i + 1] = fmaf(e, s, oc);
        }
    }
}

/* mistral/mistral_model.h:79-122 */
void ora_apply_rope(float *q, float *k, int pos, const float *theta_inv, int n_heads,
                    int n_kv_heads, int head_dim) {
    int hd2 = head_dim / 2;
    float cos_tab[128], sin_tab[128];
    float fpos = (float)pos;
    for (int i = 0; i < hd2; i++) {
        float ang = theta_inv[i] * fpos; /* vDSP_vsmul, :87-88 */
        sin_tab[i] = sinf(ang);          /* vvsincosf, :90 */
        cos_tab[i] = cosf(ang);
    }
    if (q) rope_rotate(q, n_heads, head_dim, cos_tab, sin_tab);
    if (k) rope_rotate(k, n_kv_heads, head_dim, cos_tab, sin_tab);
}

/* mistral/mistral_ane_prefill.h:177-186 */
void ora_apply_rope_batch(float *Q, float *K, int start_pos, const float *theta_inv,
                          int n_heads, int n_kv_heads, int head_dim, int S) {
    for (int t = 0; t < S; t++)
        ora_apply_rope(Q ? Q + (size_t)t * n_heads * head_dim : NULL,
                       K ? K + (size_t)t * n_kv_heads * head_dim : NULL, start_pos + t,
                       theta_inv, n_heads, n_kv_heads, head_dim);
}

/* ------------------------------------------------------------- softmax -- */

/* mistral/mistral_model.h:245-256 */
void ora_softmax_vec(float *x, int n) {
    float max_val = x[0];
    for (int i = 1; i < n; i++)
        if (x[i] > max_val) max_val = x[i];
    float neg_max = -max_val;
    for (int i = 0; i < n; i++) x[i] = x[i] + neg_max;
    for (int i = 0; i < n; i++) x[i] = expf(x[i]);
    float sum = 0.0f;
    for (int i = 0; i < n; i++) sum += x[i];
    float inv_sum = 1.0f / sum;
    for (int i = 0; i < n; i++) x[i] = x[i] * inv_sum;
}

/* ------------------------------------------------------------ KV cache -- */

/* mistral/kv_cache.h:22-35 */
int ora_kv_alloc(OraKV *c, int n_layers, int n_kv_heads, int head_dim, int max_seq) {
    c->n_layers = n_layers;
    c->n_kv_heads = n_kv_heads;
    c->head_dim = head_dim;
    c->max_seq = max_seq;
    c->kv_dim = n_kv_heads * head_dim;
    size_t sz = (size_t)n_layers * max_seq * c->kv_dim * sizeof(uint16_t);
    c->k_cache = (uint16_t *)calloc(sz, 1);
    c->v_cache = (uint16_t *)calloc(sz, 1);
    c->pos = 0;
    c->len = 0;
    return (c->k_cache && c->v_cache) ? 0 : -1;
}

/* mistral/kv_cache.h:38-42 (slot = seq_pos % max_seq at :39) */
uint16_t *ora_kv_k_at(const OraKV *c, int layer, int seq_pos) {
    int t = seq_pos % c->max_seq;
    return c->k_cache + (size_t)layer * c->max_seq * c->kv_dim + (size_t)t * c->kv_dim;
}

/* mistral/kv_cache.h:45-49 */
uint16_t *ora_kv_v_at(const OraKV *c, int layer, int seq_pos) {
    int t = seq_pos % c->max_seq;
    return c->v_cache + (size_t)layer * c->max_seq * c->kv_dim + (size_t)t * c->kv_dim;
}

/* mistral/kv_cache.h:53-57 */
void ora_kv_write(OraKV *c, int layer, int pos, const uint16_t *k_vec, const uint16_t *v_vec) {
    size_t sz = (size_t)c->kv_dim * sizeof(uint16_t);
    memcpy(ora_kv_k_at(c, layer, pos), k_vec, sz);
    memcpy(ora_kv_v_at(c, layer, pos), v_vec, sz);
}

/* mistral/kv_cache.h:61-68 */
uint16_t *ora_kv_k(const OraKV *c, int layer) {
    return c->k_cache + (size_t)layer * c->max_seq * c->kv_dim;
}
uint16_t *ora_kv_v(const OraKV *c, int layer) {
    return c->v_cache + (size_t)layer * c->max_seq * c->kv_dim;
}

/* mistral/kv_cache.h:70-75 */
void ora_kv_free(OraKV *c) {
    free(c->k_cache);
    free(c->v_cache);
    c->k_cache = NULL;
    c->v_cache = NULL;
}

/* ---------------------------------------------------- S=1 attention ----- */

/* Dot product of one pre-scaled q head with one fp16 key row, in the lane
 * order of mistral/mistral_model.h:399-441: four 4-lane accumulators, each
 * 32-wide step adding dims d+4a.. then d+16+4a.. into accumulator a; then
 * (acc0+acc1)+(acc2+acc3) lane-wise and a pairwise horizontal add. */
static float dot_s1(const float *qh, const uint16_t *kt, int hd) {
#ifdef ORA_USE_AVX2
    if ((hd & 15) == 0) return dot_avx2(qh, kt, hd);
#endif
    float acc[4][4] = {{0}};
    for (int d = 0; d < hd; d += 32) {
        for (int a = 0; a < 4; a++)
            for (int i = 0; i < 4; i++)
                acc[a][i] = fmaf(qh[d + 4 * a + i], ora_f16_to_f32(kt[d + 4 * a + i]), acc[a][i]);
        for (int a = 0; a < 4; a++)
            for (int i = 0; i < 4; i++)
                acc[a][i] = fmaf(qh[d + 16 + 4 * a + i], ora_f16_to_f32(kt[d + 16 + 4 * a + i]),
                                 acc[a][i]);
    }
    float s[4];
    for (int i = 0; i < 4; i++) {
        float s01 = acc[0][i] + acc[1][i];
        float s23 = acc[2][i] + acc[3][i];
        s[i] = s01 + s23;
    }
    return (s[0] + s[1]) + (s[2] + s[3]);
}

/* One head of mistral/mistral_model.h:386-486 (q already pre-scaled). */
static void gqa_one_head(const float *qh, float *att_h, float *oh, const uint16_t *kcache_base,
                         const uint16_t *vcache_base, int kvh, int hd, int kv_dim, int max_seq,
                         int pos) {
    int seq_len = (pos + 1 < max_seq) ? pos + 1 : max_seq; /* :367 */
    int ring = (pos + 1 > max_seq);                         /* :368 */
    int ring_off = ring ? (pos + 1 - seq_len) : 0;          /* :369 */
    for (int t = 0; t < seq_len; t++) {
        int ct = ring ? ((ring_off + t) % max_seq) : t; /* :396 */
        const uint16_t *kt = kcache_base + (size_t)ct * kv_dim + (size_t)kvh * hd;
        att_h[t] = dot_s1(qh, kt, hd);
    }
    ora_softmax_vec(att_h, seq_len); /* :445 */
    memset(oh, 0, (size_t)hd * sizeof(float));
    for (int t = 0; t < seq_len; t++) {
        float a = att_h[t];
        if (a == 0.0f) continue; /* :455 */
        int ct = ring ? ((ring_off + t) % max_seq) : t;
        const uint16_t *vt = vcache_base + (size_t)ct * kv_dim + (size_t)kvh * hd;
#ifdef ORA_USE_AVX2
        if ((hd & 7) == 0) {
            axpy_avx2(a, vt, oh, hd);
            continue;
        }
#endif
        for (int d = 0; d < hd; d++) oh[d] = fmaf(a, ora_f16_to_f32(vt[d]), oh[d]);
    }
}

/* mistral/mistral_model.h:362-487 */
void ora_gqa_attention(float *q, float *att, float *out, const uint16_t *kcache_base,
                       const uint16_t *vcache_base, int n_heads, int heads_per_kv, int hd,
                       int max_seq, int pos) {
    float inv_sqrt_hd = 1.0f / sqrtf((float)hd); /* :371 */
    for (int i = 0; i < n_heads * hd; i++) q[i] = q[i] * inv_sqrt_hd;
    int n_kv_heads = n_heads / heads_per_kv;
    int kv_dim = n_kv_heads * hd;
    for (int h = 0; h < n_heads; h++)
        gqa_one_head(q + (size_t)h * hd, att + (size_t)h * max_seq, out + (size_t)h * hd,
                     kcache_base, vcache_base, h / heads_per_kv, hd, kv_dim, max_seq, pos);
}

/* ---------------------------------------------------- S>1 attention ----- */

/* mistral/mistral_ane_prefill.h:189-204 */
void ora_kv_write_batch(OraKV *kv, int layer, int start_pos, const float *K_buf,
                        const float *V_buf, int kv_dim, int S) {
    uint16_t *k16 = (uint16_t *)malloc((size_t)kv_dim * sizeof(uint16_t));
    uint16_t *v16 = (uint16_t *)malloc((size_t)kv_dim * sizeof(uint16_t));
    for (int t = 0; t < S; t++) {
        int pos = start_pos + t;
        ora_cvt_f32_to_f16(K_buf + (size_t)t * kv_dim, k16, kv_dim);
        ora_cvt_f32_to_f16(V_buf + (size_t)t * kv_dim, v16, kv_dim);
        ora_kv_write(kv, layer, pos % kv->max_seq, k16, v16);
    }
    int end_pos = start_pos + S;
    if (end_pos > kv->len && end_pos <= kv->max_seq)
        kv->len = end_pos;
    else if (end_pos > kv->max_seq)
        kv->len = kv->max_seq;
    free(k16);
    free(v16);
}

/* Dot in the lane order of mistral/mistral_ane_prefill.h:243-250: two
 * 4-lane accumulators over 8-wide steps, then a pairwise horizontal add. */
static float dot_batch(const float *qh, const uint16_t *ks, int hd) {
#ifdef ORA_USE_AVX2
    if ((hd & 15) == 0) return dot_avx2(qh, ks, hd);
#endif
    float a0[4] = {0, 0, 0, 0}, a1[4] = {0, 0, 0, 0};
    for (int d = 0; d < hd; d += 8)
        for (int i = 0; i < 4; i++) {
            a0[i] = fmaf(qh[d + i], ora_f16_to_f32(ks[d + i]), a0[i]);
            a1[i] = fmaf(qh[d + 4 + i], ora_f16_to_f32(ks[d + 4 + i]), a1[i]);
        }
    float s[4];
    for (int i = 0; i < 4; i++) s[i] = a0[i] + a1[i];
    return (s[0] + s[1]) + (s[2] + s[3]);
}

/* One (token, head) unit of mistral/mistral_ane_prefill.h:219-273. */
static void batch_one(const float *qh, float *att_h, float *oh, const uint16_t *kbase,
                      const uint16_t *vbase, int kvh, int hd, int kv_dim, int max_seq, int pos) {
    int seq_len = pos + 1; /* :221-222 */
    if (seq_len > max_seq) seq_len = max_seq;
    float scale = 1.0f / sqrtf((float)hd); /* :236 */
    for (int s = 0; s < seq_len; s++) {
        int cache_s = s;
        if (pos + 1 > max_seq) cache_s = (pos + 1 - seq_len + s) % max_seq; /* :238-241 */
        const uint16_t *ks = kbase + (size_t)cache_s * kv_dim + (size_t)kvh * hd;
        att_h[s] = dot_batch(qh, ks, hd) * scale; /* :250 */
    }
    ora_softmax_vec(att_h, seq_len); /* :253 */
    for (int s = 0; s < seq_len; s++) {
        float a = att_h[s];
        if (a == 0) continue; /* :258 */
        int cache_s = s;
        if (pos + 1 > max_seq) cache_s = (pos + 1 - seq_len + s) % max_seq;
        const uint16_t *vs = vbase + (size_t)cache_s * kv_dim + (size_t)kvh * hd;
#ifdef ORA_USE_AVX2
        if ((hd & 7) == 0) {
            axpy_avx2(a, vs, oh, hd);
            continue;
        }
#endif
        for (int d = 0; d < hd; d++) oh[d] = fmaf(a, ora_f16_to_f32(vs[d]), oh[d]);
    }
}

/* mistral/mistral_ane_prefill.h:207-275 */
void ora_attention_batch(const float *Q, float *attn_out, const OraKV *kv, int layer,
                         int start_pos, int n_heads, int n_kv_heads, int head_dim, int S,
                         float *att_scratch) {
    int dim = n_heads * head_dim;
    int heads_per_kv = n_heads / n_kv_heads;
    int kv_dim = n_kv_heads * head_dim;
    memset(attn_out, 0, (size_t)dim * S * sizeof(float)); /* :217 */
    const uint16_t *kb = ora_kv_k(kv, layer);
    const uint16_t *vb = ora_kv_v(kv, layer);
    for (int t = 0; t < S; t++)
        for (int h = 0; h < n_heads; h++)
            batch_one(Q + (size_t)t * dim + (size_t)h * head_dim,
                      att_scratch + (size_t)h * kv->max_seq,
                      attn_out + (size_t)t * dim + (size_t)h * head_dim, kb, vb, h / heads_per_kv,
                      head_dim, kv_dim, kv->max_seq, start_pos + t);
}

/* -------------------------------------------------- step compositions -- */

/* mistral/mistral_model.h:849-863 (steps 4-6 of the decode layer) */
void ora_decode_step(OraKV *kv, int layer, float *q, float *k, const float *v, int pos,
                     const float *theta_inv, int n_heads, int n_kv_heads, float *att,
                     float *out) {
    int hd = kv->head_dim;
    int kv_dim = kv->kv_dim;
    ora_apply_rope(q, k, pos, theta_inv, n_heads, n_kv_heads, hd); /* :850 */
    uint16_t *k16 = (uint16_t *)malloc((size_t)kv_dim * sizeof(uint16_t));
    uint16_t *v16 = (uint16_t *)malloc((size_t)kv_dim * sizeof(uint16_t));
    ora_cvt_f32_to_f16(k, k16, kv_dim); /* :854-855 */
    ora_cvt_f32_to_f16(v, v16, kv_dim);
    int cache_pos = pos % kv->max_seq; /* :856 */
    ora_kv_write(kv, layer, cache_pos, k16, v16);
    if (kv->len < kv->max_seq && pos + 1 > kv->len) kv->len = pos + 1; /* :858 */
    free(k16);
    free(v16);
    ora_gqa_attention(q, att, out, ora_kv_k(kv, layer), ora_kv_v(kv, layer), n_heads,
                      n_heads / n_kv_heads, hd, kv->max_seq, pos); /* :861-863 */
}

/* mistral/speculative.h:92-101: verify = sequential S=1 decode steps */
void ora_verify_steps(OraKV *kv, int layer, float *Q, float *K, const float *V, int start_pos,
                      int S, const float *theta_inv, int n_heads, int n_kv_heads, float *att,
                      float *out) {
    int dim = n_heads * kv->head_dim;
    for (int t = 0; t < S; t++)
        ora_decode_step(kv, layer, Q + (size_t)t * dim, K + (size_t)t * kv->kv_dim,
                        V + (size_t)t * kv->kv_dim, start_pos + t, theta_inv, n_heads,
                        n_kv_heads, att, out + (size_t)t * dim);
}

/* mistral/mistral_model.h:908-1075, phases 1 and 2 without the projections,
 * Wo and the FFN.  Phase 2's loop body (:961-1044: q pre-scaled by
 * 1/sqrtf(hd), the four-accumulator dot, softmax_vec, the zero-skipping AV)
 * is the arithmetic of gqa_attention_neon (:362-487), restated above as
 * ora_gqa_attention. */
void ora_prefill_chunk_attention(OraKV *kv, int layer, float *Q, float *K, const float *V,
                                 const int *positions, int S, const float *theta_inv,
                                 int n_heads, int n_kv_heads, float *att, float *out) {
    int hd = kv->head_dim;
    int kv_dim = kv->kv_dim;
    int dim = n_heads * hd;
    int max_seq = kv->max_seq;
    uint16_t *k16 = (uint16_t *)malloc((size_t)kv_dim * sizeof(uint16_t));
    uint16_t *v16 = (uint16_t *)malloc((size_t)kv_dim * sizeof(uint16_t));
    for (int ti = 0; ti < S; ti++) { /* phase 1, :935-955 */
        int pos = positions[ti];
        float *qb = Q + (size_t)ti * dim;
        float *kb = K + (size_t)ti * kv_dim;
        ora_apply_rope(qb, kb, pos, theta_inv, n_heads, n_kv_heads, hd); /* :946 */
        ora_cvt_f32_to_f16(kb, k16, kv_dim);                              /* :949-950 */
        ora_cvt_f32_to_f16(V + (size_t)ti * kv_dim, v16, kv_dim);
        ora_kv_write(kv, layer, pos % max_seq, k16, v16);                 /* :951 */
        if (kv->len < max_seq && pos + 1 > kv->len) kv->len = pos + 1;   /* :952 */
    }
    free(k16);
    free(v16);
    for (int ti = 0; ti < S; ti++) /* phase 2, :961-1044 */
        ora_gqa_attention(Q + (size_t)ti * dim, att, out + (size_t)ti * dim, ora_kv_k(kv, layer),
                          ora_kv_v(kv, layer), n_heads, n_heads / n_kv_heads, hd, max_seq,
                          positions[ti]);
}

/* tests/test_cpu_ref.h:113-147 */
void ora_ref_gqa_attention(float *out, const float *q, const float *k, const float *v, int S,
                           int n_heads, int n_kv_heads, int head_dim) {
    float scale = 1.0f / sqrtf((float)head_dim);
    int gqa_ratio = n_heads / n_kv_heads;
    float *scores = (float *)malloc((size_t)S * sizeof(float));
    for (int h = 0; h < n_heads; h++) {
        int kv_h = h / gqa_ratio;
        for (int t = 0; t < S; t++) {
            float mx = -1e30f;
            for (int s = 0; s <= t; s++) {
                float dot = 0;
                for (int d = 0; d < head_dim; d++)
                    dot += q[(size_t)t * n_heads * head_dim + h * head_dim + d] *
                           k[(size_t)s * n_kv_heads * head_dim + kv_h * head_dim + d];
                scores[s] = dot * scale;
                if (scores[s] > mx) mx = scores[s];
            }
            float sm = 0;
            for (int s = 0; s <= t; s++) {
                scores[s] = expf(scores[s] - mx);
                sm += scores[s];
            }
            float inv = 1.0f / sm;
            for (int s = 0; s <= t; s++) scores[s] *= inv;
            for (int d = 0; d < head_dim; d++) {
                float val = 0;
                for (int s = 0; s <= t; s++)
                    val += scores[s] * v[(size_t)s * n_kv_heads * head_dim + kv_h * head_dim + d];
                out[(size_t)t * n_heads * head_dim + h * head_dim + d] = val;
            }
        }
    }
    free(scores);
}

/* ------------------------------------------------ CPU baseline drivers -- */

int ora_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void ora_decode_layers(const float *Q, float *out, const uint16_t *k_cache,
                       const uint16_t *v_cache, int n_layers, int n_heads, int heads_per_kv,
                       int hd, int max_seq, int pos, int n_threads) {
    int n_kv = n_heads / heads_per_kv;
    int kv_dim = n_kv * hd;
    size_t layer_stride = (size_t)max_seq * kv_dim;
    float inv_sqrt_hd = 1.0f / sqrtf((float)hd);
    int n_units = n_layers * n_heads;
#ifdef _OPENMP
    int nt = n_threads > 0 ? n_threads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        float *att = (float *)malloc((size_t)max_seq * sizeof(float));
        float *qh = (float *)malloc((size_t)hd * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 1)
#endif
        for (int u = 0; u < n_units; u++) {
            int l = u / n_heads, h = u % n_heads;
            const float *src = Q + (size_t)l * n_heads * hd + (size_t)h * hd;
            for (int d = 0; d < hd; d++) qh[d] = src[d] * inv_sqrt_hd;
            gqa_one_head(qh, att, out + (size_t)l * n_heads * hd + (size_t)h * hd,
                         k_cache + l * layer_stride, v_cache + l * layer_stride, h / heads_per_kv,
                         hd, kv_dim, max_seq, pos);
        }
        free(att);
        free(qh);
    }
    (void)n_threads;
}

void ora_attention_batch_layers(const float *Q, float *out, const uint16_t *k_cache,
                                const uint16_t *v_cache, int n_layers, int n_heads,
                                int n_kv_heads, int hd, int max_seq, int start_pos, int S,
                                int n_threads) {
    int heads_per_kv = n_heads / n_kv_heads;
    int kv_dim = n_kv_heads * hd;
    int dim = n_heads * hd;
    size_t layer_stride = (size_t)max_seq * kv_dim;
    long n_units = (long)n_layers * S * n_heads;
    memset(out, 0, (size_t)n_layers * S * dim * sizeof(float));
#ifdef _OPENMP
    int nt = n_threads > 0 ? n_threads : omp_get_max_threads();
#pragma omp parallel num_threads(nt)
#endif
    {
        float *att = (float *)malloc((size_t)max_seq * sizeof(float));
#ifdef _OPENMP
#pragma omp for schedule(dynamic, 4)
#endif
        for (long u = 0; u < n_units; u++) {
            int l = (int)(u / ((long)S * n_heads));
            int rem = (int)(u % ((long)S * n_heads));
            int t = rem / n_heads, h = rem % n_heads;
            size_t off = ((size_t)l * S + t) * dim + (size_t)h * hd;
            batch_one(Q + off, att, out + off, k_cache + l * layer_stride,
                      v_cache + l * layer_stride, h / heads_per_kv, hd, kv_dim, max_seq,
                      start_pos + t);
        }
        free(att);
    }
    (void)n_threads;
}
