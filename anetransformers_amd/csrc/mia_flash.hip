// mia_flash.hip -- S>1 causal GQA attention on fp16 MFMA for gfx950.
//
// Replaces mistral/mistral_ane_prefill.h:207-275 (attention_batch) and, with
// staged drafts, the sequential verify of mistral/speculative.h:92-101.
//
// Rows of a tile are (query t, head g) pairs of one kv head, row = t*G + g, so
// the G query heads of a group share every K/V tile.  One wave owns 32 rows.
// Per 64-key tile (staged in LDS):
//   S^T[key][row] = K . Q^T   v_mfma_f32_32x32x16_f16, A = K rows from LDS,
//                             B = Q^T held in registers for the whole loop
//   online softmax per row    each lane owns one row (the D column), so the
//                             running max/sum/rescale stay lane-local
//   O^T[dim][row] += V^T . P^T  P^T feeds the B operand straight from the
//                             S^T accumulator layout (same key permutation on
//                             both operands); V^T is gathered from LDS.
// Query t at position start+t attends the window [pos-L+1, pos], L =
// min(pos+1, max_seq) (mistral_ane_prefill.h:220-241); positions >= start come
// from the staging buffer when one is given, which keeps the ring untouched
// until the caller commits (sequential-verify semantics on a wrapped ring).
// Key ranges are split over workgroups; a second kernel merges the partials
// (log-sum-exp).
#include "mia_device.h"
#include "mia_kernels.h"

namespace mia {

namespace {

constexpr int kKeys = 64;                // keys per LDS tile
constexpr int kPitch = HD + 8;           // LDS row pitch in halfs (272 B)

struct FlashSmem {
  _Float16 k[kKeys][kPitch];
  _Float16 v[kKeys][kPitch];
};

__device__ __forceinline__ int window_lo(int pos, int max_seq) {
  // pos - min(pos+1, M) + 1
  return pos + 1 > max_seq ? pos + 1 - max_seq : 0;
}

template <int G, int NW>
__global__ void __launch_bounds__(64 * NW) flash_kernel(FlashParams p) {
  constexpr int RT = 32 * NW;  // rows per tile
  constexpr int NT = 64 * NW;
  __shared__ FlashSmem sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int half = lane >> 5;
  const int col = lane & 31;
  const int kvh = blockIdx.x % p.n_kv;
  const int rest = blockIdx.x / p.n_kv;
  const int rtile = rest % p.n_rtiles;
  const int split = rest / p.n_rtiles;
  const int kv_dim = p.n_kv * HD;
  const int dim_model = p.n_kv * G * HD;

  // This lane's row.
  const int row0 = rtile * RT;
  const int row = row0 + w * 32 + col;
  const int t = row / G;
  const int g = row % G;
  const bool row_valid = t < p.S;
  const int pos_t = p.start_pos + (row_valid ? t : p.S - 1);
  const int lo_t = window_lo(pos_t, p.max_seq);
  const int hi_t = pos_t;

  // Key range of the tile and of this split.
  const int t0 = row0 / G;
  const int t1 = min((row0 + RT - 1) / G, p.S - 1);
  const int klo = window_lo(p.start_pos + t0, p.max_seq);
  const int khi = p.start_pos + t1;
  const int ks = klo + split * p.split_keys;
  const int ke = min(ks + p.split_keys, khi + 1);

  // Q^T operand: col = row, k = dims 16*st + 8*half .. +8, scaled, fp16.
  h8 qb[8];
  {
    const float *qsrc = p.Q + (size_t)(row_valid ? t : 0) * dim_model + (size_t)(kvh * G + g) * HD;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const f4 *src = reinterpret_cast<const f4 *>(qsrc + 16 * st + 8 * half);
      f4 a = src[0], b = src[1];
      float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) qb[st][e] = (_Float16)(row_valid ? v[e] * p.qscale : 0.f);
    }
  }

  f16v o[4];
#pragma unroll
  for (int db = 0; db < 4; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o[db][i] = 0.f;
  float m_run = -INFINITY, l_run = 0.f;

  for (int kb = ks; kb < ke; kb += kKeys) {
    // Cooperative K/V tile load: 64 keys x 16 chunks of 16 B per tensor.
    for (int c = tid; c < kKeys * 16; c += NT) {
      const int kr = c >> 4, cc = c & 15;
      const int kp = min(kb + kr, ke - 1);  // absolute key position (clamped)
      const _Float16 *ksrc;
      const _Float16 *vsrc;
      if (p.kstage != nullptr && kp >= p.start_pos) {
        size_t off = (size_t)(kp - p.start_pos) * kv_dim + (size_t)kvh * HD + 8 * cc;
        ksrc = p.kstage + off;
        vsrc = p.vstage + off;
      } else {
        int slot = kp % p.max_seq;
        size_t off = (size_t)slot * kv_dim + (size_t)kvh * HD + 8 * cc;
        ksrc = p.kc + off;
        vsrc = p.vc + off;
      }
      *reinterpret_cast<u4 *>(&sm.k[kr][8 * cc]) = *reinterpret_cast<const u4 *>(ksrc);
      *reinterpret_cast<u4 *>(&sm.v[kr][8 * cc]) = *reinterpret_cast<const u4 *>(vsrc);
    }
    __syncthreads();

    // S^T for two 32-key blocks.
    f16v s[2];
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s[kb2][i] = 0.f;
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        h8 a = *reinterpret_cast<const h8 *>(&sm.k[32 * kb2 + col][16 * st + 8 * half]);
        s[kb2] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[st], s[kb2], 0, 0, 0);
      }
    }

    // Mask + online softmax (lane-local row state).
    float mloc = -INFINITY;
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb + 32 * kb2 + (i >> 2) * 8 + 4 * half + (i & 3);
        const bool ok = row_valid && key >= lo_t && key <= hi_t && key < ke;
        s[kb2][i] = ok ? s[kb2][i] : -INFINITY;
        mloc = fmaxf(mloc, s[kb2][i]);
      }
    mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
    const float m_new = fmaxf(m_run, mloc);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m_run - m_use);
    float lsum = 0.f;
    h8 pb[4];  // P^T B operands: 2 blocks x 2 k-steps
#pragma unroll
    for (int kb2 = 0; kb2 < 2; ++kb2)
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float pv = fast_exp2(s[kb2][i] - m_use);
        lsum += pv;
        pb[kb2 * 2 + (i >> 3)][i & 7] = (_Float16)pv;
      }
    l_run = l_run * alpha + lsum;
    m_run = m_new;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o[db][i] *= alpha;

    // O^T += V^T P^T.  k-step ks4 covers keys 16*ks4 .. +16; this half's 8
    // keys are {0-3, 8-11} + 4*half within it (the S^T row permutation).
#pragma unroll
    for (int ks4 = 0; ks4 < 4; ++ks4) {
      const int kbase = 16 * ks4 + 4 * half;
#pragma unroll
      for (int db = 0; db < 4; ++db) {
        const int dim = 32 * db + col;
        h8 a;
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = sm.v[kbase + (e >> 2) * 8 + (e & 3)][dim];
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, pb[ks4], o[db], 0, 0, 0);
      }
    }
    __syncthreads();
  }

  const float l_tot = l_run + __shfl_xor(l_run, 32);
  // O^T layout: lane holds row `row` (column of D) and dims
  // 32*db + (i/4)*8 + 4*half + (i%4).
  if (p.nsplit == 1) {
    if (row_valid) {
      float *dst = p.out + (size_t)t * dim_model + (size_t)(kvh * G + g) * HD;
      const float inv = 1.0f / l_tot;
#pragma unroll
      for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int i4 = 0; i4 < 4; ++i4) {
          f4 v = {o[db][4 * i4 + 0] * inv, o[db][4 * i4 + 1] * inv, o[db][4 * i4 + 2] * inv,
                  o[db][4 * i4 + 3] * inv};
          *reinterpret_cast<f4 *>(dst + 32 * db + 8 * i4 + 4 * half) = v;
        }
    }
    return;
  }

  // Split partials: [tile][split][RT][128] and [tile][split][RT] (m, l).
  const size_t tile_id = (size_t)kvh * p.n_rtiles + rtile;
  const size_t pb_idx = (tile_id * p.nsplit + split) * RT + (w * 32 + col);
  {
    float *dst = p.part_o + pb_idx * HD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4) {
        f4 v = {o[db][4 * i4 + 0], o[db][4 * i4 + 1], o[db][4 * i4 + 2], o[db][4 * i4 + 3]};
        *reinterpret_cast<f4 *>(dst + 32 * db + 8 * i4 + 4 * half) = v;
      }
    if (half == 0)
      *reinterpret_cast<float2 *>(p.part_ml + pb_idx * 2) = make_float2(m_run, l_tot);
  }
}

// Split-K merge: one workgroup per 8 rows of a tile, thread = (row, 4 dims).
// A separate launch, so the kernel boundary orders the partial writes before
// these reads (no agent-scope fence in the attention kernel).
template <int G>
__global__ void __launch_bounds__(256) flash_merge_kernel(FlashParams p, int rt) {
  const int tid = threadIdx.x;
  const int blocks_per_tile = rt / 8;
  const int tile_id = blockIdx.x / blocks_per_tile;
  const int rl = (blockIdx.x % blocks_per_tile) * 8 + tid / 32;
  const int d4 = tid % 32;
  const int kvh = tile_id / p.n_rtiles, rtile = tile_id % p.n_rtiles;
  const int row = rtile * rt + rl;
  const int t = row / G, g = row % G;
  if (t >= p.S) return;
  const int dim_model = p.n_kv * G * HD;
  float M = -INFINITY;
  for (int sp = 0; sp < p.nsplit; ++sp)
    M = fmaxf(M, p.part_ml[(((size_t)tile_id * p.nsplit + sp) * rt + rl) * 2]);
  float Ls = 0.f;
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < p.nsplit; ++sp) {
    const size_t idx = ((size_t)tile_id * p.nsplit + sp) * rt + rl;
    float2 ml = *reinterpret_cast<const float2 *>(p.part_ml + idx * 2);
    float e = fast_exp2(ml.x - M);
    Ls = __builtin_fmaf(e, ml.y, Ls);
    f4 v = *reinterpret_cast<const f4 *>(p.part_o + idx * HD + 4 * d4);
    acc += e * v;
  }
  *reinterpret_cast<f4 *>(p.out + (size_t)t * dim_model + (size_t)(kvh * G + g) * HD + 4 * d4) =
      acc * (1.0f / Ls);
}

}  // namespace

size_t flash_scratch_bytes(int n_kv, int n_rtiles, int nsplit, int rows_per_tile) {
  return (size_t)n_kv * n_rtiles * nsplit * rows_per_tile * (HD + 2) * sizeof(float);
}

void flash_plan(int S, int n_kv, int G, int start_pos, int max_seq, int target_wgs, int *n_rtiles,
                int *nsplit, int *split_keys, int *rows_per_tile) {
  const int rows = S * G;
  const int rt = rows <= 32 ? 32 : 128;
  const int ntiles = (rows + rt - 1) / rt;
  // Widest key range over the tiles (the last tile reaches the furthest).
  long maxkeys = 0;
  for (int ti = 0; ti < ntiles; ++ti) {
    int t0 = (ti * rt) / G;
    int t1 = ((ti + 1) * rt - 1) / G;
    if (t1 > S - 1) t1 = S - 1;
    long p0 = (long)start_pos + t0;
    long lo = p0 + 1 > max_seq ? p0 + 1 - max_seq : 0;
    long hi = (long)start_pos + t1;
    if (hi - lo + 1 > maxkeys) maxkeys = hi - lo + 1;
  }
  long want_splits = (target_wgs + (long)n_kv * ntiles - 1) / ((long)n_kv * ntiles);
  if (want_splits < 1) want_splits = 1;
  long sk = (maxkeys + want_splits - 1) / want_splits;
  sk = ((sk + kKeys - 1) / kKeys) * kKeys;
  if (sk < 256) sk = 256;
  long ns = (maxkeys + sk - 1) / sk;
  if (ns < 1) ns = 1;
  *n_rtiles = ntiles;
  *nsplit = (int)ns;
  *split_keys = (int)sk;
  *rows_per_tile = rt;
}

hipError_t launch_flash(const FlashParams &p, int G, hipStream_t s, int *rows_per_tile_out) {
  if (G != 4) return hipErrorInvalidValue;
  const int rows = p.S * G;
  const int rt = rows <= 32 ? 32 : 128;
  if (rows_per_tile_out) *rows_per_tile_out = rt;
  dim3 grid(p.n_kv * p.n_rtiles * p.nsplit);
  if (rt == 32)
    hipLaunchKernelGGL((flash_kernel<4, 1>), grid, dim3(64), 0, s, p);
  else
    hipLaunchKernelGGL((flash_kernel<4, 4>), grid, dim3(256), 0, s, p);
  if (p.nsplit > 1)
    hipLaunchKernelGGL((flash_merge_kernel<4>), dim3(p.n_kv * p.n_rtiles * (rt / 8)), dim3(256), 0,
                       s, p, rt);
  return hipGetLastError();
}

}  // namespace mia
