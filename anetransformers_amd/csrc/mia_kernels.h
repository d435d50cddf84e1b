// mia_kernels.h -- host-side launch interface of the attention kernels.
// Only the C-ABI shim (mia_capi.cpp) calls these; no torch types anywhere.
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>
#include <stddef.h>
#include <stdint.h>

namespace mia {

// Per-device set-up, called by mia_init with the device current: raises the
// dynamic LDS limit of the kernels that use more than 64 KB.
hipError_t prepare_flash();
hipError_t prepare_gemm();

// S=1 split-K flash-decode over the fp16 sequence-major ring of one layer.
struct DecodeParams {
  const float *q;          // [n_kv*G][128] fp32: raw (fused) or already rotated
  const float *knew;       // [n_kv][128] fp32 raw new key (fused only)
  const float *vnew;       // [n_kv][128] fp32 new value (fused only)
  const float *theta_inv;  // [64] (fused only)
  _Float16 *kc;            // layer base [max_seq][kv_dim]
  _Float16 *vc;
  float *out;              // [n_kv*G][128]
  _Float16 *new_k;         // fused: where the new token's fp16 k / v rows go
  _Float16 *new_v;         // ([kv_dim] each); null: ring slot new_slot
  float *part_o;           // [n_kv][nchunk][G][128] unnormalised partial outputs
  float *part_ml;          // [n_kv][nchunk][G][2] partial (max, sum), log2 domain
  int max_seq;             // ring capacity M
  int pos;                 // absolute position of the query token
  int L;                   // window length min(pos+1, M)
  int start;               // slot of the oldest window entry, (pos+1-L) mod M
  int new_slot;            // pos mod M
  int n_kv;
  int nchunk;              // workgroups per kv head (chunks of whole 16-key tiles)
  float qscale;            // (1/sqrt(128)) * log2(e)
  // kDecodePositions: n_tok tokens, token t at positions[t] (device int32);
  // q, out [n_tok][n_kv*G][128], partials per token; pos / L / start unused.
  // theta_inv set: q is rotated in-kernel at the token's position.
  const int *positions;
  int n_tok;
};
enum { kDecodePlain = 0, kDecodeFused = 1, kDecodePositions = 2 };

// Scratch needed by launch_decode for a given shape (bytes of part_o+part_ml).
size_t decode_scratch_bytes(int n_kv, int G, int nchunk, int n_tok = 1);
int decode_pick_nchunk(int L, int n_kv, int target_wgs);
// Main kernel only; launch_decode_merge adds the cross-chunk merge (nchunk > 1).
// ev0/ev1 (may be null) are stamped at the kernel's start and end.
hipError_t launch_decode(const DecodeParams &p, int G, int mode, hipStream_t s, hipEvent_t ev0,
                         hipEvent_t ev1);
hipError_t launch_decode_merge(const DecodeParams &p, hipStream_t s);

// S>=1 causal attention on fp16 MFMA for the queries start_pos..start_pos+S-1.
struct FlashParams {
  const float *Q;          // [S][n_heads*128] fp32 (scale applied in-kernel)
  const float *rope_cs;    // [S][64] (cos, sin) of the query positions: rotate Q
                           // in-kernel; nullptr: Q already rotated
  const _Float16 *kc;      // layer base [max_seq][kv_dim]
  const _Float16 *vc;
  const _Float16 *kstage;  // [S][kv_dim] staged new keys (nullptr: all keys in ring)
  const _Float16 *vstage;
  float *out;              // [S][n_heads*128]
  float *part_o;           // split-K partials (nsplit > 1)
  float *part_ml;
  _Float16 *commit_k;      // nsplit > 1 with staged drafts: the merge kernel copies
  _Float16 *commit_v;      // the staged rows into these ring layers (else null)
  int S, n_kv, max_seq, start_pos;
  int n_rtiles;            // row tiles per kv head
  int nsplit;              // key splits per row tile
  int split_keys;          // keys per split (multiple of 64)
  float qscale;
};
size_t flash_scratch_bytes(int n_kv, int n_rtiles, int nsplit, int rows_per_tile);
// Main kernel only; launch_flash_merge adds the split merge (nsplit > 1).
// ev0/ev1 (may be null) are stamped at the kernel's start and end.
hipError_t launch_flash(const FlashParams &p, int G, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1);
hipError_t launch_flash_merge(const FlashParams &p, hipStream_t s);
void flash_plan(int S, int n_kv, int G, int start_pos, int max_seq, int target_wgs,
                int *n_rtiles, int *nsplit, int *split_keys, int *rows_per_tile);

// Elementwise helpers.
hipError_t launch_rope(float *q, float *k, int S, int start_pos, const float *theta_inv,
                       int n_heads, int n_kv, hipStream_t s);
// K rotated and K, V rounded to fp16 into a dense staging buffer or the ring;
// cs_out (may be null) receives the [S][64] (cos, sin) table of the positions.
hipError_t launch_rope_to_f16(const float *K, const float *V, const float *theta_inv, int S,
                              int start_pos, int n_kv, _Float16 *kdst, _Float16 *vdst,
                              float *cs_out, hipStream_t s);
hipError_t launch_rope_to_ring(const float *K, const float *V, const float *theta_inv, int S,
                               int start_pos, int n_kv, _Float16 *kc, _Float16 *vc, int max_seq,
                               float *cs_out, hipStream_t s);
hipError_t launch_kv_write(_Float16 *kc, _Float16 *vc, const float *K, const float *V, int S,
                           int start_pos, int max_seq, int kv_dim, hipStream_t s);
// The chunked prefill's phase 1 (mistral_model.h:935-955) for the K / V side:
// token t's k rotated at positions[t] (device int32), k and v rounded to fp16
// and written to slot positions[t] % max_seq unless a later token of the
// chunk takes the same slot (the reference's in-order writes leave the last).
// owner: null (each token scans the later ones, O(S^2) reads: short chunks)
// or an int32 [max_seq] area holding -1 everywhere, left so (linear in S).
hipError_t launch_rope_kv_positions(const float *K, const float *V, const float *theta_inv,
                                    const int *positions, int S, int n_kv, _Float16 *kc,
                                    _Float16 *vc, int max_seq, int *owner, hipStream_t s);
// Staged rows 0..S-1 -> ring slots (start_pos + t) % max_seq, for n_layers
// layers ring_stride / stage_stride elements apart.
hipError_t launch_commit(_Float16 *kc, _Float16 *vc, const _Float16 *kst, const _Float16 *vst,
                         int S, int start_pos, int max_seq, int kv_dim, hipStream_t s,
                         int n_layers = 1, size_t ring_stride = 0, size_t stage_stride = 0);
hipError_t launch_fill_normal(_Float16 *dst, size_t n, uint64_t seed, hipStream_t s);

// Peak microbenchmarks (mia_peaks.hip).
hipError_t launch_peak_read_stream(const void *buf, size_t bytes, int num_cus, hipStream_t s);
hipError_t launch_peak_read_ring(const _Float16 *kc, const _Float16 *vc, int n_kv, int max_seq,
                                 int L, int start, int nchunk, hipStream_t s);
hipError_t launch_peak_mfma_f16(int iters, int num_cus, double *flop, hipStream_t s);
// An empty kernel of the given grid; ev0/ev1 (may be null) stamped at its
// start and end like the attention kernels' profile events.
hipError_t launch_peak_empty(int workgroups, int threads, hipStream_t s, hipEvent_t ev0,
                             hipEvent_t ev1);

// W4A8 projections (mistral/dequant.h).  x [nblocks*32] fp32, 16-byte aligned
// -> nblocks Q8_0 blocks of 36 bytes.
hipError_t launch_quantize_q8_0(const float *x, uint8_t *out, int nblocks, hipStream_t s);
// y = W . x for up to three Q4_0 matrices stacked as virtual rows (w0's rows,
// then w1's, then w2's); bpr = blocks per row, even; pointers 4-byte aligned.
// x is either Q8_0 blocks (x) or fp32 values quantised in-kernel (xf, 16-byte
// aligned, bpr * 32 <= kQ4MaxFusedInDim; the C-ABI's fp32-input matvecs take
// up to kQ4MaxF32InDim).
constexpr int kQ4MaxF32InDim = 8192;
struct Q4MatvecParams {
  const uint8_t *w0, *w1, *w2;
  float *y0, *y1, *y2;
  const uint8_t *x;  // Q8_0 blocks [bpr], or null when xf is set
  const float *xf;   // fp32 [bpr * 32], or null
  int rows0;         // rows of w0
  int rows01;        // rows of w0 + w1
  int total_rows;    // rows of w0 + w1 + w2
  int bpr;
  // The decode layer's steps around a matvec, with xf only (each null when
  // unused): rms_w: xf is RMS-normalised first, (xf * (1 / sqrtf(mean(xf^2) +
  // eps))) * rms_w, as launch_rmsnorm does it; up: xf is the FFN gate and
  // the input is gate * (1 / (1 + expf(-gate))) * up; resid: y = resid[row] +
  // the row's sum (resid may be y itself).
  const float *rms_w;
  float eps;
  const float *up;
  const float *resid;
  // swiglu: w0 (gate) and w1 (up) of rows0 rows each, their rows interleaved
  // (virtual row 2j is w0's row j, 2j + 1 is w1's) so that one wave holds
  // both sums of row j and writes y0[j] = gate * (1 / (1 + expf(-gate))) * up
  // (total_rows = 2 * rows0; rows01, y1, y2 unused).
  int swiglu;
};
constexpr int kQ4MaxFusedInDim = 16384;
hipError_t launch_q4_matvec(const Q4MatvecParams &p, hipStream_t s, hipEvent_t ev0,
                            hipEvent_t ev1);
hipError_t launch_scale_rows(_Float16 *base, long n_rows, int row_elems, int every, int offset,
                             float factor, hipStream_t s);

// Prefill layer pieces (mia_prefill.hip).  Y[S][N] = A[S][K] . W^T with W up
// to three Q4_0 matrices stacked as virtual rows (as Q4MatvecParams); K a
// multiple of 64; A 16-byte aligned with lda a multiple of 4.
enum { kGemmStore = 0, kGemmAdd = 1, kGemmSiluMul = 2 };
struct GemmParams {
  // the fp32 activations as fp16 hi + lo planes, [S][K] each (launch_split_hilo)
  const _Float16 *ahi, *alo;
  const uint8_t *w0, *w1, *w2;
  int rows0, rows01, N;  // rows of w0, of w0 + w1, and in all
  int K, S;
  // kGemmStore: y0 [S][rows0], y1 [S][rows01 - rows0], y2 [S][N - rows01];
  // kGemmAdd: y0 [S][N] += result; kGemmSiluMul: y0 [S][N] holds the gate and
  // becomes gate * sigmoid(gate) * result.
  float *y0, *y1, *y2;
  // K split over blockIdx.z (1: none).  With ksplit > 1 the partial products
  // go to part [ksplit][S][N] and a second kernel sums them in split order
  // and applies the epilogue.
  int ksplit;
  float *part;
  // kGemmSiluMul only: when set, the result goes out as fp16 hi + lo planes
  // [S][N] (the next GEMM's input, launch_split_hilo's split) instead of
  // into y0.
  _Float16 *ohi, *olo;
  // w0, w1, w2 in the GEMM tile layout of launch_q4_pack (row counts and K
  // multiples of 64) instead of the GGUF layout
  int packed;
};
long gemm_tiles(int N, int S);
// Q4_0 [N][K / 32] in the GGUF layout -> the GEMM tile layout (same size;
// N and K multiples of 64, src 4-byte and dst 16-byte aligned, no overlap).
hipError_t launch_q4_pack(const void *src, void *dst, int N, int K, hipStream_t s);
int gemm_pick_ksplit(int N, int K, int S, int num_cus);
hipError_t launch_q4_gemm(const GemmParams &p, int mode, int num_cus, hipStream_t s,
                          hipEvent_t ev0, hipEvent_t ev1);
// x [n] fp32 -> hi, lo [n] fp16 with x = hi + lo to ~2^-22 (n a multiple of 8).
hipError_t launch_split_hilo(const float *x, long n, _Float16 *hi, _Float16 *lo, int num_cus,
                             hipStream_t s);
// The same rows written as fp16 hi + lo planes (launch_split_hilo's split).
hipError_t launch_rmsnorm_split(_Float16 *hi, _Float16 *lo, const float *in, const float *w,
                                int dim, int S, float eps, hipStream_t s);
hipError_t launch_rmsnorm(float *out, const float *in, const float *w, int dim, int S, float eps,
                          hipStream_t s);

// Weight types by GGML id (mia_kquant.hip).  Rows of `cols` weights, cols a
// multiple of 32 (256 for Q4_K / Q6_K); W 16-byte aligned for F32 / F16 /
// Q4_K, 2-byte for Q4_0 / Q6_K; fp32 x 16-byte aligned, Q8_0 x 4-byte.
enum { kTypeF32 = 0, kTypeF16 = 1, kTypeQ40 = 2, kTypeQ4K = 12, kTypeQ6K = 14 };
long typed_row_bytes(int type, int cols);  // 0: type or cols not supported
// y [rows] = W . x with x fp32 [cols] or (x_q8) Q8_0 blocks [cols / 32].
hipError_t launch_typed_matvec(const void *W, int type, const void *x, bool x_q8, float *y,
                               int rows, int cols, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1);
// out [rows][cols] fp32 = the weights the reference multiplies.
hipError_t launch_typed_dequant(const void *W, int type, float *out, int rows, int cols,
                                hipStream_t s);
// The weights as the fp16 GEMM operands: hi [rows][cols]; for types whose
// values are not fp16 (Q6_K, F32) also lo [rows][cols] and rscale [rows], with
// w = (hi + lo) * rscale to 2^-22 relative (lo, rscale unused otherwise).
bool typed_is_f16_exact(int type);
hipError_t launch_typed_split(const void *W, int type, _Float16 *hi, _Float16 *lo, float *rscale,
                              int rows, int cols, hipStream_t s);
// Y [S][N] (+)= rscale[n] * ((C1[s][n] + C1[S + s][n]) + C2[s][n]); C2 and
// rscale null: Y (+)= C1[s][n] + C1[S + s][n].
hipError_t launch_hilo_combine(const float *C1, const float *C2, const float *rscale, float *Y,
                               int S, int N, bool add, hipStream_t s);
// The decode layer's residual steps (mia_layer.hip): x += y, then out =
// rmsnorm(x) (dim a multiple of 4, pointers 16-byte aligned); x += y.
hipError_t launch_residual_rmsnorm(float *x, const float *y, const float *w, float *out, int dim,
                                   float eps, hipStream_t s);
hipError_t launch_add(float *x, const float *y, int n, hipStream_t s);
// gate [n] = gate * sigmoid(gate) * up (the SwiGLU product).
hipError_t launch_silu_mul(float *gate, const float *up, long n, hipStream_t s);

// The decode layer's Q4_K / Q6_K matvecs with their neighbouring steps
// inside: up to three matrices of one input (each of type kTypeQ4K or
// kTypeQ6K), their rows stacked as virtual rows (w[0]'s, then w[1]'s, then
// w[2]'s).  The fp32 input xf [cols] (16-byte aligned, cols a multiple of 256
// up to kKqLayerMaxCols) is RMS-normalised (when rms_w is set: (xf * (1 /
// sqrtf(mean(xf^2) + eps))) * rms_w, launch_rmsnorm's arithmetic) and
// quantised to Q8_0 blocks (launch_quantize_q8_0's) by every workgroup, so
// each row's sum equals launch_typed_matvec's on the separately formed
// blocks, bit for bit.  Epilogues: y = resid[row] + sum (resid may be y), or
// swiglu: w[0] (gate) and w[1] (up) of rows[0] rows each, interleaved so that
// one wave holds row j of both and writes y[0][j] = gate * (1 / (1 +
// expf(-gate))) * up.  rows[0] and rows[0] + rows[1] must be multiples of the
// workgroup's rows (launch_kq_layer_matvec checks it).
constexpr int kKqLayerMaxCols = 16384;
struct KqLayerParams {
  const void *w[3];
  int type[3];
  float *y[3];
  int rows[3];
  int cols;
  const float *xf;
  const float *rms_w;
  float eps;
  const float *resid;
  int swiglu;
};
hipError_t launch_kq_layer_matvec(const KqLayerParams &p, hipStream_t s, hipEvent_t ev0,
                                  hipEvent_t ev1);

}  // namespace mia
