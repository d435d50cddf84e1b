/*
 * miattn.h -- C ABI of libmiattn.so: the MI355X (gfx950) Mistral-7B GQA
 * attention hot path.  Plain pointers and sizes only.
 *
 * Conventions
 *   - Every function returns 0 (MIA_OK) or a nonzero mia_status; the message
 *     of the last failure on the calling thread is in mia_last_error().
 *   - "dev" pointers are device memory (mia_malloc or any hipMalloc'd
 *     memory); fp16 tensors are IEEE binary16 bit patterns (uint16_t).
 *   - stream is a hipStream_t, or NULL for the library's stream on the
 *     current device.  Kernels are enqueued asynchronously; outputs are valid
 *     after mia_stream_sync(stream).
 *   - Shapes: head_dim must be 128 and n_heads / n_kv_heads must be 4 (the
 *     Mistral-7B GQA ratio); other shapes return MIA_ERR_UNSUPPORTED.
 *   - KV ring layout (mistral/kv_cache.h:2-4): per layer
 *     [max_seq][n_kv_heads][head_dim] fp16; position p lives in slot
 *     p % max_seq (mistral/kv_cache.h:39).  k_layer / v_layer point at a
 *     layer base (kv_k / kv_v, mistral/kv_cache.h:61-68).
 *   - Calls that use device scratch (the split-K partials of the attention
 *     and GEMM kernels, the GEMM's fp16 hi / lo activation planes) share one
 *     per-device area of each kind: calls that overlap on one device
 *     (several host threads, or several streams) race.  The first call at a new size may allocate (not inside a HIP
 *     graph capture: warm up first).
 */
#ifndef MIATTN_H
#define MIATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    MIA_OK = 0,
    MIA_ERR_INVALID = 1,     /* bad argument */
    MIA_ERR_UNSUPPORTED = 2, /* shape the gfx950 kernels are not built for */
    MIA_ERR_HIP = 3,         /* HIP runtime error (message in mia_last_error) */
    MIA_ERR_NO_DEVICE = 4    /* no HIP device / library not initialised */
} mia_status;

/* ---- runtime plumbing -------------------------------------------------- */
int mia_init(int device);            /* select device, create stream; idempotent */
int mia_device_count(int *count);
const char *mia_last_error(void);
int mia_version(void);               /* 100 * major + minor */
int mia_malloc(void **dptr, size_t bytes);
int mia_free(void *dptr);
int mia_memcpy_h2d(void *dst_dev, const void *src_host, size_t bytes);
int mia_memcpy_d2h(void *dst_host, const void *src_dev, size_t bytes);
int mia_memcpy_d2d(void *dst_dev, const void *src_dev, size_t bytes);
int mia_memset(void *dst_dev, int value, size_t bytes);
int mia_stream_create(void **stream);
int mia_stream_destroy(void *stream);
int mia_stream_sync(void *stream);
int mia_device_sync(void);
int mia_event_create(void **event);
int mia_event_destroy(void *event);
int mia_event_record(void *event, void *stream);
int mia_event_elapsed_ms(float *ms, void *start, void *stop);

/* Opt-in kernel timing on the current device: while on, the main kernel of
 * every attention call is launched with a HIP event pair that the dispatch
 * stamps at its start and end (kind 0: the S=1 decode kernel of
 * mia_gqa_attention / mia_decode_step / mia_attention_step with S=1; kind 1:
 * the S>1 flash kernel; kind 2: the Q4_0 matvec kernel of mia_q4_0_matvec /
 * mia_q4_0_matvec_qkv; kind 3: the Q4_0 GEMM kernel of mia_q4_0_gemm_f32 /
 * mia_prefill_layer; kind 4: the empty kernel of mia_peak_empty, mia_peaks.h;
 * kind 5: the matvec kernel of mia_matvec_f32 / mia_matvec_q8 for types
 * other than Q4_0);
 * merge, quantize, RMSNorm and RoPE kernels are not timed.
 * mia_profile_end stops recording, synchronises and returns the number of
 * timed launches of that kind and their summed duration. */
int mia_profile_begin(void);
int mia_profile_end(int kind, int *count, double *total_ms);

/* ---- synthetic inputs (benchmark) --------------------------------------- */
/* dst[i] = fp16(N(0,1)) from a counter-based splitmix64 + Box-Muller stream. */
int mia_fill_normal_f16(uint16_t *dst_dev, size_t n, uint64_t seed, void *stream);
/* Multiply rows offset, offset+every, ... (row_elems fp16 each) by factor. */
int mia_scale_rows_f16(uint16_t *base_dev, long n_rows, int row_elems, int every, int offset,
                       float factor, void *stream);

/* ---- hot path ------------------------------------------------------------ */

/* In-place adjacent-pair RoPE of S tokens at positions start_pos + t.
 * Replaces apply_rope (mistral/mistral_model.h:79-122) for S = 1 and
 * apply_rope_batch (mistral/mistral_ane_prefill.h:177-186).
 * q [S][n_heads*128] fp32 dev (may be NULL), k [S][n_kv_heads*128] (may be
 * NULL), theta_inv [64] dev (precompute_rope_theta, mistral_model.h:69-74). */
int mia_rope_f32(float *q, float *k, int S, int start_pos, const float *theta_inv, int n_heads,
                 int n_kv_heads, int head_dim, void *stream);

/* fp32 -> fp16 (RNE) and ring write of S tokens at slots (start_pos+t) %
 * max_seq.  Replaces kv_write_batch (mistral/mistral_ane_prefill.h:189-204;
 * the caller keeps the len bookkeeping).  K, V [S][kv_dim] fp32 dev. */
int mia_kv_write_f32(uint16_t *k_layer, uint16_t *v_layer, const float *K, const float *V, int S,
                     int start_pos, int max_seq, int kv_dim, void *stream);

/* S=1 GQA attention over the ring as it stands.  Replaces gqa_attention_neon
 * (mistral/mistral_model.h:362-487): window = last min(pos+1, max_seq)
 * positions, oldest first; scale 1/sqrt(128).  q [n_heads*128] fp32 dev,
 * already rotated (not modified); out [n_heads*128] fp32 dev.  The
 * reference's att scratch is not used. */
int mia_gqa_attention(const float *q, float *out, const uint16_t *k_layer,
                      const uint16_t *v_layer, int n_heads, int heads_per_kv, int hd,
                      int max_seq, int pos, void *stream);

/* Steps 4-6 of the decode layer (mistral/mistral_model.h:849-863) fused in
 * one launch: RoPE(q, k) at pos, fp16 round of k and v, ring write at
 * pos % max_seq, S=1 attention (the new token attended from its fp16 copy).
 * q [n_heads*128], k, v [n_kv_heads*128] raw fp32 dev (not modified);
 * theta_inv [64] dev; out [n_heads*128] fp32 dev. */
int mia_decode_step(const float *q, const float *k, const float *v, const float *theta_inv,
                    uint16_t *k_layer, uint16_t *v_layer, float *out, int n_heads,
                    int n_kv_heads, int hd, int max_seq, int pos, void *stream);

/* mia_decode_step with no device allocation.  No counterpart in the
 * reference: this is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  The
 * split-K partials go to a fixed per-device area in the library
 * (4,259,840 bytes: 256 chunks at 8 kv heads; more kv heads get fewer chunks
 * rather than an error), set up by mia_init, which must have been called on
 * the device first (MIA_ERR_NO_DEVICE otherwise).  Results are those of
 * mia_decode_step.  Every call on a device shares that area: calls that
 * overlap on one device (several host threads or streams) race.  The call
 * makes no hipMalloc / hipFree and is not timed by mia_profile_*. */
int mia_decode_step_noalloc(const float *q, const float *k, const float *v,
                            const float *theta_inv, uint16_t *k_layer, uint16_t *v_layer,
                            float *out, int n_heads, int n_kv_heads, int hd, int max_seq, int pos,
                            void *stream);

/* S>=1 causal GQA attention over the ring as it stands, query t at position
 * start_pos + t.  Replaces attention_batch (mistral/mistral_ane_prefill.h:
 * 207-275).  Q [S][n_heads*128] fp32 dev, rotated; out [S][n_heads*128]. */
int mia_attention_batch(const float *Q, float *out, const uint16_t *k_layer,
                        const uint16_t *v_layer, int n_heads, int n_kv_heads, int hd,
                        int max_seq, int start_pos, int S, void *stream);

/* Attention of S tokens, each at its own position over the ring as it
 * stands: token t attends the window [pos-L+1, pos], L = min(pos+1, max_seq),
 * pos = positions[t] -- phase 2 of mistral_layer_prefill_chunk
 * (mistral/mistral_model.h:961-1044), which is gqa_attention_neon per token.
 * Q [S][n_heads*128] fp32 dev, rotated; positions [S] int32 dev (any order,
 * >= 0; a negative position gives a zero row); out [S][n_heads*128].
 * 1 <= S <= 65535.  Each token reads its own window, so contiguous runs of
 * positions are cheaper through mia_attention_batch. */
int mia_attention_positions(const float *Q, float *out, const uint16_t *k_layer,
                            const uint16_t *v_layer, const int *positions, int n_heads,
                            int n_kv_heads, int hd, int max_seq, int S, void *stream);

/* The attention of mistral_layer_prefill_chunk (mistral/mistral_model.h:
 * 908-1075), phases 1 and 2: every token's k rotated at positions[t], k and v
 * rounded to fp16 and written to slot positions[t] % max_seq (in token order:
 * a later token in the same slot wins), then mia_attention_positions over the
 * ring so written, with q rotated at positions[t].  Q [S][n_heads*128], K, V
 * [S][n_kv_heads*128] raw fp32 dev (not modified); theta_inv [64] dev.  The
 * caller keeps the len bookkeeping (mistral_model.h:952).  Chunks of more
 * than 64 tokens use a per-device int32 [max_seq] area (allocated on first
 * use) to find each slot's last token in one pass. */
int mia_attention_chunk(const float *Q, const float *K, const float *V, const int *positions,
                        const float *theta_inv, uint16_t *k_layer, uint16_t *v_layer, float *out,
                        int n_heads, int n_kv_heads, int hd, int max_seq, int S, void *stream);

/* S tokens through steps 4-6 with sequential semantics: the result equals S
 * calls of mia_decode_step at start_pos, start_pos+1, ... (the verify loop of
 * mistral/speculative.h:92-101), also when the ring has wrapped: drafts are
 * staged during attention and committed to their slots afterwards.
 * Q [S][n_heads*128], K, V [S][n_kv_heads*128] raw fp32 dev (not modified). */
int mia_attention_step(const float *Q, const float *K, const float *V, const float *theta_inv,
                       uint16_t *k_layer, uint16_t *v_layer, float *out, int n_heads,
                       int n_kv_heads, int hd, int max_seq, int start_pos, int S, void *stream);

/* The verify step without touching the ring: the result equals S calls of
 * mia_decode_step at start_pos, start_pos+1, ... (as mia_attention_step), but
 * the S rotated fp16 keys and values are left in k_stage / v_stage
 * [S][n_kv_heads*128] (device) and the ring is only read.  After acceptance,
 * mia_commit_staged writes the accepted drafts.  Replaces the per-layer body of
 * spec_verify (mistral/speculative.h:92-101) so that rejected drafts never
 * reach the ring: the reference leaves them in their slots
 * (speculative.h:336-341), which on a wrapped ring are the oldest positions
 * of the next step's window.  16-byte aligned pointers. */
int mia_attention_step_staged(const float *Q, const float *K, const float *V,
                              const float *theta_inv, const uint16_t *k_layer,
                              const uint16_t *v_layer, uint16_t *k_stage, uint16_t *v_stage,
                              float *out, int n_heads, int n_kv_heads, int hd, int max_seq,
                              int start_pos, int S, void *stream);

/* Writes staged rows 0..n_keep-1 (n_keep <= S_staged) to ring slots
 * (start_pos + t) % max_seq, for n_layers layers at once: k_cache / v_cache
 * are layer 0's ring (layers max_seq*kv_dim elements apart, kv_cache.h:2-4)
 * and k_stage / v_stage hold [n_layers][S_staged][kv_dim]. */
int mia_commit_staged(uint16_t *k_cache, uint16_t *v_cache, const uint16_t *k_stage,
                      const uint16_t *v_stage, int n_layers, int S_staged, int n_keep,
                      int start_pos, int max_seq, int kv_dim, void *stream);

/* ---- W4A8 projections either side of the attention step ------------------ */
/* Block formats of mistral/dequant.h: Q4_0 = 18 bytes per 32 weights (fp16
 * scale, 16 bytes of nibbles: byte j low = weight j, high = weight j+16, each
 * stored + 8; dequant.h:17-31); Q8_0 = 36 bytes per 32 values (fp32 scale,
 * 32 int8; dequant.h:535-541).  A Q4_0 matrix [out_dim][in_dim] is out_dim
 * rows of in_dim/32 blocks, as GGUF stores it. */

/* x [n] fp32 dev (16-byte aligned, n a multiple of 32) -> n/32 Q8_0 blocks
 * (4-byte aligned).  Replaces quantize_f32_to_q8_0 (mistral/dequant.h:
 * 545-612): d = amax/127, q = round-half-even(x * (1/d)) saturated, d = 0 and q = 0
 * for an all-zero block; bit-identical to it. */
int mia_quantize_q8_0(const float *x, void *out_q8, int n, void *stream);

/* y [out_dim] fp32 = W (Q4_0) . x_q8.  Replaces q4_matvec_sdot_parallel for
 * Q4_0 weights (mistral/mistral_model.h:649-668 -> q4_0_q8_0_matvec_sdot_parallel,
 * mistral/dequant.h:1022-1137), used for Wo at mistral_model.h:866-867.
 * in_dim must be a multiple of 64 (an even number of blocks per row, as every
 * Mistral-7B projection has); W, x_q8, y 4-byte aligned device memory.  Block
 * terms are rounded as the reference's; their sum is reassociated. */
int mia_q4_0_matvec(const void *W, const void *x_q8, float *y, int out_dim, int in_dim,
                    void *stream);

/* The Q, K and V projections against one quantised input in one launch.
 * Replaces q4_matvec_sdot_parallel_fused_qkv (mistral/mistral_model.h:676-745,
 * called at :840-842): yq [dim] = Wq . x, yk [kv_dim] = Wk . x,
 * yv [kv_dim] = Wv . x, each row as in mia_q4_0_matvec. */
int mia_q4_0_matvec_qkv(const void *Wq, const void *Wk, const void *Wv, const void *x_q8,
                        float *yq, float *yk, float *yv, int dim, int kv_dim, int in_dim,
                        void *stream);

/* quantize_f32_to_q8_0 followed by the matvec, as the decode layer calls
 * them (mistral/mistral_model.h:866-867 for Wo; :833-842 for Q, K, V), in one
 * launch: x [in_dim] fp32 dev, 16-byte aligned, in_dim <= 8192.  Every
 * workgroup forms the Q8_0 blocks of x in LDS with mia_quantize_q8_0's
 * arithmetic, so y is bit-identical to mia_quantize_q8_0 + mia_q4_0_matvec
 * (resp. _qkv); the blocks themselves are not written out. */
int mia_q4_0_matvec_f32(const void *W, const float *x, float *y, int out_dim, int in_dim,
                        void *stream);
int mia_q4_0_matvec_qkv_f32(const void *Wq, const void *Wk, const void *Wv, const float *x,
                            float *yq, float *yk, float *yv, int dim, int kv_dim, int in_dim,
                            void *stream);

/* The FFN's gate and up projections against one quantised input in one
 * launch.  Replaces q4_matvec_sdot_parallel_fused_pair (mistral/
 * mistral_model.h:750-811, called at :880-885): y1 [out_dim] = W1 . x,
 * y3 [out_dim] = W3 . x, each row as in mia_q4_0_matvec; the _f32 form
 * quantises x inside the launch as mia_q4_0_matvec_f32 does (in_dim <= 8192,
 * bit-identical to mia_quantize_q8_0 + mia_q4_0_matvec_pair). */
int mia_q4_0_matvec_pair(const void *W1, const void *W3, const void *x_q8, float *y1, float *y3,
                         int out_dim, int in_dim, void *stream);
int mia_q4_0_matvec_pair_f32(const void *W1, const void *W3, const float *x, float *y1,
                             float *y3, int out_dim, int in_dim, void *stream);

/* ---- the rest of the prefill layer ---------------------------------------- */

/* rmsnorm_batch (mistral/mistral_ane_prefill.h:163-175): out[t] = in[t] *
 * (1/sqrt(mean(in[t]^2) + eps)) * w for S rows of dim fp32 (dev, 16-byte
 * aligned, dim a multiple of 4).  out may equal in. */
int mia_rmsnorm_f32(float *out, const float *in, const float *w, int dim, int S, float eps,
                    void *stream);

/* tiled_q4_gemm for Q4_0 weights (mistral/mistral_ane_prefill.h:1018-1042,
 * dequantise + cblas_sgemm): Y[S][out_dim] = X[S][in_dim] . W^T, fp32 X and Y
 * (dev, 16-byte aligned), in_dim a multiple of 64.  fp16 MFMA on X split into
 * hi + lo halves (per-device scratch of S * in_dim * 4 bytes) with the block
 * scales applied in fp32: within fp32 rounding of the reference's sums, not
 * bit-identical to them.  Range: the hi half is fp16, so every |x| must be
 * below 65504 (larger values give non-finite outputs, where the reference's
 * fp32 product stays finite); below 2^-3 the lo half is subnormal and x is
 * carried to 2^-25 absolute rather than 2^-22 relative.  The same holds for
 * every GEMM input of mia_prefill_layer (the RMSNorm outputs, the attention
 * output and the SwiGLU product). */
int mia_q4_0_gemm_f32(const void *W, const float *X, float *Y, int out_dim, int in_dim, int S,
                      void *stream);

/* The same weights regrouped once, at load time, for the GEMM (no reference
 * counterpart: the reference dequantises the GGUF blocks per 128-row tile,
 * mistral/mistral_ane_prefill.h:1018-1042; the values are unchanged).  Wp
 * (dev, 16-byte aligned, not overlapping W) receives the out_dim x in_dim / 32
 * blocks of W (dev, 4-byte aligned) in the GEMM tile layout: for each 64 rows
 * and 64 columns one contiguous 2,304-byte tile, the rows' quant bytes first,
 * their fp16 scales after.  out_dim and in_dim multiples of 64. */
int mia_q4_0_pack_gemm(const void *W, void *Wp, int out_dim, int in_dim, void *stream);

/* mia_q4_0_gemm_f32 on weights in the tile layout of mia_q4_0_pack_gemm:
 * bit-identical results, fewer and contiguous weight loads.  out_dim a
 * multiple of 64, Wp 16-byte aligned. */
int mia_q4_0_gemm_packed_f32(const void *Wp, const float *X, float *Y, int out_dim, int in_dim,
                             int S, void *stream);

/* One layer's Q4_0 weights on the device (GGUF layout) and RMSNorm weights. */
typedef struct {
    const void *wq, *wk, *wv, *wo; /* attention projections */
    const void *w1, *w2, *w3;      /* gate, down, up */
    const float *rms_att, *rms_ffn;
} mia_layer_weights;

/* blas_prefill_layer (mistral/mistral_ane_prefill.h:1081-1110) on the GPU:
 * X [S][dim] fp32 dev is updated in place (X += attention(...) . Wo^T, then
 * X += SwiGLU(...) . W2^T), the layer's ring gets the S rotated fp16 K/V at
 * slots (start_pos + t) % max_seq.  dim = n_heads * 128, hidden and dim
 * multiples of 64.  The attention step is the reference's
 * apply_rope_batch + kv_write_batch + attention_batch (:1096-1098): all S
 * tokens' K/V are written first (a token that a later token of the chunk
 * overwrites writes nothing, as the in-order writes leave it), then every
 * query attends the ring as it then stands, so when a chunk wraps the ring
 * earlier tokens see later tokens' K/V in recycled slots, as the reference's
 * do.  (mia_attention_step instead has the sequential-verify semantics.)
 * Activations live in a per-device work area (58 MB at S = 512). */
int mia_prefill_layer(float *X, const mia_layer_weights *lw, const float *theta_inv,
                      uint16_t *k_layer, uint16_t *v_layer, int dim, int hidden, int n_heads,
                      int n_kv_heads, float eps, int max_seq, int start_pos, int S,
                      void *stream);

/* mia_prefill_layer with the seven Q4_0 matrices of lw in the tile layout of
 * mia_q4_0_pack_gemm (16-byte aligned; the RMSNorm weights as before):
 * bit-identical results. */
int mia_prefill_layer_packed(float *X, const mia_layer_weights *lw, const float *theta_inv,
                             uint16_t *k_layer, uint16_t *v_layer, int dim, int hidden,
                             int n_heads, int n_kv_heads, float eps, int max_seq, int start_pos,
                             int S, void *stream);

/* ---- weight types: Q4_K, Q6_K, F16, F32 beside Q4_0 ----------------------- */
/* GGML type ids (mistral/gguf_loader.h:32-38).  Q4_K = 144 bytes per 256
 * weights (fp16 d, fp16 dmin, 12 bytes of 6-bit sub-block scales and mins,
 * 128 bytes of nibbles; mistral/dequant.h:23-29); Q6_K = 210 bytes per 256
 * weights (ql[128], qh[64], int8 scales[16], fp16 d; dequant.h:283-289).  A
 * matrix [out_dim][in_dim] is out_dim rows of in_dim / 32 (Q4_0) or in_dim /
 * 256 (Q4_K, Q6_K) blocks, or of in_dim values, as GGUF stores it.  in_dim
 * must be a multiple of 32 (256 for the K-quants); W is device memory,
 * 16-byte aligned for F32 / F16 / Q4_K, 2-byte aligned for Q4_0 / Q6_K. */
enum {
    MIA_TYPE_F32 = 0,
    MIA_TYPE_F16 = 1,
    MIA_TYPE_Q4_0 = 2,
    MIA_TYPE_Q4_K = 12,
    MIA_TYPE_Q6_K = 14
};

/* Bytes of one row of in_dim weights of the type; 0 for a type or in_dim
 * the library does not take (q_row_bytes, mistral/mistral_ane_prefill.h:
 * 1008-1015). */
long mia_weight_row_bytes(int type, int in_dim);

/* out [rows][cols] fp32 dev (16-byte aligned) = the weights the reference
 * multiplies, bit for bit (dequant_weight_to_fp32_buf, mistral/
 * mistral_ane_prefill.h:907-1000): Q4_K through the fp16 arithmetic of
 * dequant_q4_K_block_neon (dequant.h:68-125), Q6_K as dequant_q6_K_block
 * (dequant.h:291-307), Q4_0 as d * (q - 8) in fp32. */
int mia_dequant_f32(const void *W, int type, float *out, int rows, int cols, void *stream);

/* y [out_dim] = W . x with fp32 x (dev, 16-byte aligned): q4_matvec /
 * q4_matvec_parallel (mistral/mistral_model.h:211-243, 581-644) for every
 * type.  The weights are those of mia_dequant_f32, multiplied and summed in
 * fp32 (the reference's sgemv / NEON lane sums, in another order). */
int mia_matvec_f32(const void *W, int type, const float *x, float *y, int out_dim, int in_dim,
                   void *stream);

/* q4_matvec_sdot_parallel for every type (mistral/mistral_model.h:649-670):
 * Q4_0 is mia_q4_0_matvec (in_dim a multiple of 64); the other types take
 * x as the Q8_0 blocks' values d * q in fp32, as the reference does, and
 * multiply as mia_matvec_f32. */
int mia_matvec_q8(const void *W, int type, const void *x_q8, float *y, int out_dim, int in_dim,
                  void *stream);

/* tiled_q4_gemm for every type (mistral/mistral_ane_prefill.h:1018-1042):
 * Y[S][out_dim] = X[S][in_dim] . W^T, fp32 X and Y (dev, 16-byte aligned).
 * Q4_0 is mia_q4_0_gemm_f32.  The other types multiply on fp16 MFMA with fp32
 * accumulation (hipBLASLt; the algorithm of each GEMM shape is timed and
 * picked on the shape's first call in the process, which therefore waits for
 * the stream once; later calls of the shape reuse it, so repeated calls give
 * bit-identical results), within fp32 rounding of the reference's
 * dequantise + cblas_sgemm: X is split into fp16 hi + lo halves, as for Q4_0;
 * Q4_K and F16 weights are fp16 values and enter exactly; Q6_K and F32
 * weights are scaled per row by a power of two and split into hi + lo halves
 * (2^-22 relative).  Per-device work areas: out_dim * in_dim * 2 bytes
 * (twice that for Q6_K / F32), 12 * S * out_dim bytes and a 64 MiB GEMM
 * workspace.  Range as
 * mia_q4_0_gemm_f32's: every |x| below 65504, below 2^-3 carried to 2^-25
 * absolute. */
int mia_gemm_f32(const void *W, int type, const float *X, float *Y, int out_dim, int in_dim,
                 int S, void *stream);

/* The same weights converted once, at load time, into the GEMM's operand form
 * (no reference counterpart; the reference dequantises per call,
 * mistral/mistral_ane_prefill.h:1018-1042), so that the per-call conversion
 * drops out: results are bit-identical to mia_gemm_f32's in the same process
 * (the same GEMM algorithm for the shape).  Q4_0 is
 * mia_q4_0_pack_gemm's tile layout (out_dim and in_dim multiples of 64, the
 * size of the GGUF form); Q4_K and F16 become their fp16 values [out_dim]
 * [in_dim] (4x / 1x the Q4_K / F16 bytes); Q6_K and F32 the row-scaled fp16
 * hi and lo halves and the row scales.  mia_gemm_pack_bytes gives the size
 * (0 for a shape the GEMM does not take); Wp is 16-byte aligned device memory
 * not overlapping W. */
size_t mia_gemm_pack_bytes(int type, int out_dim, int in_dim);
int mia_gemm_pack(const void *W, int type, void *Wp, int out_dim, int in_dim, void *stream);
/* mia_gemm_f32 on a packed matrix. */
int mia_gemm_packed_f32(const void *Wp, int type, const float *X, float *Y, int out_dim,
                        int in_dim, int S, void *stream);

/* One layer's weights with their types (LayerWeights, mistral/
 * mistral_model.h:16-28). */
typedef struct {
    const void *wq, *wk, *wv, *wo, *w1, *w2, *w3;
    int wq_type, wk_type, wv_type, wo_type, w1_type, w2_type, w3_type;
    const float *rms_att, *rms_ffn;
} mia_layer_weights_typed;

/* blas_prefill_layer (mistral/mistral_ane_prefill.h:1081-1110) with each
 * matrix of its own type, as mia_prefill_layer otherwise (same arguments,
 * attention step and ring semantics).  A layer whose seven matrices are all
 * Q4_0 is mia_prefill_layer; any other mix multiplies each matrix as
 * mia_gemm_f32 does for its type, with the activations in fp32 and the
 * SwiGLU product
 * gate * (1 / (1 + exp(-gate))) * up (silu_mul_neon, mistral_model.h:
 * 174-199) in between. */
int mia_prefill_layer_typed(float *X, const mia_layer_weights_typed *lw, const float *theta_inv,
                            uint16_t *k_layer, uint16_t *v_layer, int dim, int hidden,
                            int n_heads, int n_kv_heads, float eps, int max_seq, int start_pos,
                            int S, void *stream);

/* mia_prefill_layer_typed with the seven matrices in mia_gemm_pack's form
 * (16-byte aligned; the types as before): bit-identical results. */
int mia_prefill_layer_typed_packed(float *X, const mia_layer_weights_typed *lw,
                                   const float *theta_inv, uint16_t *k_layer, uint16_t *v_layer,
                                   int dim, int hidden, int n_heads, int n_kv_heads, float eps,
                                   int max_seq, int start_pos, int S, void *stream);

/* ---- the decode layer ------------------------------------------------------ */
/* silu_mul_neon (mistral/mistral_model.h:174-199): gate[i] = gate[i] *
 * (1 / (1 + exp(-gate[i]))) * up[i] for n fp32 (dev) values, the SwiGLU
 * product of both layers' FFN; exp is the GPU's (within ulps of libm's). */
int mia_silu_mul_f32(float *gate, const float *up, long n, void *stream);

/* mistral_layer_decode_parallel (mistral/mistral_model.h:818-899) on the GPU
 * for the token at pos: x [dim] fp32 dev (16-byte aligned) is updated in
 * place, the layer's ring gets the token's rotated fp16 K / V at slot
 * pos % max_seq (the caller keeps kv->len, as the reference's caller does).
 * Steps and their arithmetic as the reference's: RMSNorm; x quantised to
 * Q8_0 once for Q, K and V (one fused launch when all three are Q4_0,
 * mia_q4_0_matvec_qkv_f32; otherwise each by type as mia_matvec_q8);
 * mia_decode_step; the attention output quantised for Wo; x += Wo . a; RMSNorm
 * (one launch with the residual add); gate and up (mia_q4_0_matvec_pair_f32
 * when both are Q4_0); gate * sigmoid(gate) * up; its Q8_0 blocks for W2;
 * x += W2 . h.  Weights in the GGUF layout with their types
 * (mia_layer_weights_typed); dim = n_heads * 128.  The vectors live in a
 * per-device work area (~190 KB at Mistral-7B's sizes). */
int mia_decode_layer(float *x, const mia_layer_weights_typed *lw, const float *theta_inv,
                     uint16_t *k_layer, uint16_t *v_layer, int dim, int hidden, int n_heads,
                     int n_kv_heads, float eps, int max_seq, int pos, void *stream);

/* ---- KV-ring snapshots (no counterpart in the reference) ------------------ */
/* The rings of all layers (k_cache / v_cache: device memory holding
 * [n_layers][max_seq][n_kv_heads][head_dim] fp16 each, the KVCache arrays of
 * mistral/kv_cache.h:10-20) with the cache's sizes and its pos / len cursors,
 * as one host byte string for saving and resuming a session.  Little-endian:
 * a 64-byte header ("MIAKVRG1", u32 64, u32 2, the seven int fields of
 * KVCache in its order: n_layers, n_kv_heads, head_dim, max_seq, kv_dim, pos,
 * len; u32 0; u64 bytes of one array; u64 0), then k_cache's bytes, then
 * v_cache's, each exactly as it lies in memory.  Synchronous. */

/* Bytes of a snapshot of this shape (0 for a non-positive size). */
size_t mia_kv_snapshot_bytes(int n_layers, int n_kv_heads, int head_dim, int max_seq);

/* Writes the snapshot into dst (host, dst_bytes >= mia_kv_snapshot_bytes). */
int mia_kv_snapshot_save(void *dst, size_t dst_bytes, const uint16_t *k_cache,
                         const uint16_t *v_cache, int n_layers, int n_kv_heads, int head_dim,
                         int max_seq, int pos, int len);

/* Reads a snapshot into rings of the same shape (MIA_ERR_INVALID when the
 * header is not a snapshot's, the shape differs or src is truncated); pos and
 * len (may be NULL) receive the saved cursors. */
int mia_kv_snapshot_load(const void *src, size_t src_bytes, uint16_t *k_cache, uint16_t *v_cache,
                         int n_layers, int n_kv_heads, int head_dim, int max_seq, int *pos,
                         int *len);

/* The header's fields (any output may be NULL); no device work. */
int mia_kv_snapshot_info(const void *src, size_t src_bytes, int *n_layers, int *n_kv_heads,
                         int *head_dim, int *max_seq, int *pos, int *len);

#ifdef __cplusplus
}
#endif
#endif
