// mia_flash.hip -- S>1 causal GQA attention on fp16 MFMA for gfx950.
//
// Replaces mistral/mistral_ane_prefill.h:207-275 (attention_batch) and, with
// staged drafts, the sequential verify of mistral/speculative.h:92-101.
//
// Rows are (query t, head g) pairs of one kv head, row = t*G + g, so the G
// query heads of a group share every K/V tile.  A workgroup holds SL row slabs
// of 32 rows and KH key groups; wave w works on slab w % SL over the key range
// of group w / SL, and the KH partial results are merged in LDS at the end.
// K/V tiles go from global memory straight into LDS (global_load_lds, no
// register staging), double-buffered per key group; the tile loop is software
// pipelined so that the scores of tile i+1 are computed on MFMA while the
// exponentials of tile i are formed.  Per 32-key tile:
//   S^T[key][row] = K . Q^T   v_mfma_f32_32x32x16_f16, A = K rows from LDS
//                             (ds_read_b128), B = Q^T held in registers
//   online softmax per row    each lane owns one row (the D column), so the
//                             running max / sum / rescale stay lane-local
//   O^T[dim][row] += V^T . P^T  P^T is the B operand straight from the S^T
//                             accumulator (same key permutation on both
//                             operands); V^T comes from the row-major V tile
//                             by the transposing LDS read ds_read_b64_tr_b16.
// Query t at position start+t attends the window [pos-L+1, pos], L =
// min(pos+1, max_seq) (mistral_ane_prefill.h:220-241); positions >= start come
// from the staging buffer when one is given, which keeps the ring untouched
// until the caller commits (sequential-verify semantics on a wrapped ring).
// With p.theta_inv set, the adjacent-pair RoPE of Q (mistral_model.h:79-122)
// is applied while the Q operand is built.  Masks are applied only to tiles
// that cross a window edge of the slab.  Very long key ranges over few rows
// are additionally split over workgroups and merged by a second kernel.
#include "mia_device.h"
#include "mia_kernels.h"

namespace mia {

namespace {

constexpr int kKT = 32;         // keys per tile
// K/V tiles live in LDS unpadded, one 256 B row per key, with the 16-byte
// chunk c of row r stored at chunk c ^ swz(r): rows r..r+15 then hit distinct
// bank groups for the K operand reads (same chunk, 16 rows), and the 4 rows x
// 2 chunks of a transposing V read are distinct too.
__device__ __forceinline__ int swz(int r) { return ((r & 7) << 1) | ((r >> 3) & 1); }

template <int SL, int KH>
struct FlashLayout {
  static constexpr int kTileHalfs = kKT * HD;
  // [KH][2 buffers][K, V] tiles
  static constexpr size_t kTiles = (size_t)KH * 2 * 2 * kTileHalfs * sizeof(_Float16);
  static constexpr size_t kRope = (size_t)8 * SL * 64 * sizeof(float2);
  // after the loop the tile area holds [KH][SL][32 rows][HD] partial outputs
  // and [KH][SL][32][2] (max, sum)
  static constexpr size_t kMerge = (size_t)KH * SL * 32 * (HD + 2) * sizeof(float);
  static constexpr size_t kBytes = (kTiles > kMerge ? kTiles : kMerge) + kRope;
};

__device__ __forceinline__ int window_lo(int pos, int max_seq) {
  // pos - min(pos+1, M) + 1
  return pos + 1 > max_seq ? pos + 1 - max_seq : 0;
}

typedef short s4 __attribute__((ext_vector_type(4)));
// LDS (address space 3) pointers: 32-bit addressing, no generic-pointer checks.
typedef __attribute__((address_space(3))) _Float16 lds_half;
typedef __attribute__((address_space(3))) s4 lds_s4;
typedef __attribute__((address_space(3))) h8 lds_h8;

// Four consecutive keys k0..k0+3 of dim d0 + (lane % 16) from a swizzled
// [key][128] fp16 tile: input lane i of each 16-lane group points at
// (k0 + i/4, d0 + 4*(i%4)); the transposing read returns, in output lane j,
// elements (k0 + e, d0 + j) for e = 0..3.
__device__ __forceinline__ h4 read_vt4(lds_half *tile, int k0, int d0, int lane) {
  const int i = lane & 15;
  const int r = k0 + (i >> 2);
  const int c = (d0 >> 3) + ((i & 3) >> 1);
  lds_half *src = tile + r * HD + 8 * (c ^ swz(r)) + 4 * (i & 1);
  s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s4 *)src);
  return __builtin_bit_cast(h4, v);
}

// 16 bytes per lane from global memory straight into LDS: lane i's data
// lands at byte 16*i of the wave's 1 KB block at `l` (wave-uniform).  Inline
// assembly, so that the compiler neither orders later LDS reads of the other
// buffer behind it nor waits for it; completion is awaited explicitly (vmcnt)
// before the workgroup barrier that publishes the tile.
__device__ __forceinline__ void lds_dma16(const void *g, lds_half *l) {
  const unsigned m = __builtin_amdgcn_readfirstlane((unsigned)(__UINTPTR_TYPE__)l);
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %0, off" ::"v"(g),
      "s"(m)
      : "m0");
}
// Same with a wave-uniform base address and a per-lane 32-bit byte offset.
__device__ __forceinline__ void lds_dma16_sb(const void *base, unsigned voff, lds_half *l) {
  const unsigned m = __builtin_amdgcn_readfirstlane((unsigned)(__UINTPTR_TYPE__)l);
  asm volatile(
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %0, %1" ::"v"(voff),
      "s"(base), "s"(m)
      : "m0");
}

// Issues this wave's share of the direct loads of one tensor (K or V) of the
// 32-key tile kb..kb+31 (range ending at ke) into the tile buffer dst.  A tile
// of 32 consecutive ring slots takes a uniform base plus the lane's constant
// offset; tiles that wrap or reach into the staging buffer take per-lane
// addresses.
template <int IPW, int SL>
__device__ __forceinline__ void load_tensor(const _Float16 *ring, const _Float16 *stage, int kb,
                                            int ke, int start_pos, int max_seq, int kv_dim,
                                            const int *lane_row, const int *lane_off,
                                            const unsigned *lane_boff, int slab, lds_half *dst) {
  const bool full = kb + kKT <= ke;
  const int slot0 = kb % max_seq;  // uniform, once per tile
  const bool contiguous =
      full && slot0 + kKT <= max_seq && (stage == nullptr || kb + kKT <= start_pos);
  if (contiguous) {
    const _Float16 *base = ring + (size_t)slot0 * kv_dim;
#pragma unroll
    for (int j = 0; j < IPW; ++j) lds_dma16_sb(base, lane_boff[j], dst + (slab + SL * j) * 4 * HD);
    return;
  }
#pragma unroll
  for (int j = 0; j < IPW; ++j) {
    const int r = lane_row[j];
    const int kp = min(kb + r, ke - 1);
    const bool staged = stage != nullptr && kp >= start_pos;
    int slot = slot0 + (kp - kb);
    slot = slot >= max_seq ? slot - max_seq : slot;
    const _Float16 *src = (staged ? stage : ring) +
                          (size_t)(staged ? kp - start_pos : slot) * kv_dim + lane_off[j];
    lds_dma16(src, dst + (slab + SL * j) * 4 * HD);
  }
}

template <int G, int SL, int KH>
__global__ void __launch_bounds__(64 * SL * KH) flash_kernel(FlashParams p) {
  using Lay = FlashLayout<SL, KH>;
  constexpr int NW = SL * KH;
  constexpr int RT = 32 * SL;     // rows per workgroup
  constexpr int QT = RT / G;      // queries per workgroup
  extern __shared__ __attribute__((aligned(16))) char smem[];
  lds_half *tiles = (lds_half *)smem;
  float2 *rope = reinterpret_cast<float2 *>(smem + (Lay::kBytes - Lay::kRope));

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int slab = w % SL;
  const int kg = w / SL;
  const int half = lane >> 5;
  const int col = lane & 31;
  const int kvh = blockIdx.x % p.n_kv;
  const int rest = blockIdx.x / p.n_kv;
  const int rtile = rest % p.n_rtiles;
  const int split = rest / p.n_rtiles;
  const int kv_dim = p.n_kv * HD;
  const int dim_model = p.n_kv * G * HD;

  // This lane's row and its window.
  const int row0 = rtile * RT;
  const int row = row0 + slab * 32 + col;
  const int t = row / G;
  const int g = row % G;
  const bool row_valid = t < p.S;
  const int pos_t = p.start_pos + (row_valid ? t : p.S - 1);
  const int lo_t = window_lo(pos_t, p.max_seq);
  const int hi_t = pos_t;
  // Slab-uniform bounds: keys in [lo_max, hi_min] are inside every row's window.
  const int ts0 = (row0 + slab * 32) / G;
  const int ts1 = (row0 + slab * 32 + 31) / G;
  const bool slab_full = ts1 < p.S;
  const int lo_max = window_lo(p.start_pos + min(ts1, p.S - 1), p.max_seq);
  const int hi_min = p.start_pos + ts0;

  // Key range of the workgroup (one split), then of this key group.
  const int tq0 = row0 / G;
  const int tq1 = min((row0 + RT - 1) / G, p.S - 1);
  const int klo = window_lo(p.start_pos + tq0, p.max_seq);
  const int khi = p.start_pos + tq1;
  const int ks = klo + split * p.split_keys;
  const int ke = min(ks + p.split_keys, khi + 1);
  const int nt = ke > ks ? (ke - ks + kKT - 1) / kKT : 0;
  const int g_first = (int)((long)kg * nt / KH);
  const int g_count = (int)((long)(kg + 1) * nt / KH) - g_first;
  const int n_iter = (nt + KH - 1) / KH;

  // Tile buffers (per key group: K ring and V ring of 2) and this lane's
  // share of the direct loads.  One wave instruction moves 4 keys (64 lanes x
  // 16 B); the SL waves of a key group share the 8 instructions per tensor of
  // a 32-key tile.  Lane i of instruction j loads key row 4j + i/16, logical
  // chunk (i%16) ^ swz(row), which the hardware writes at byte 16*i of the
  // instruction's 1 KB block.
  constexpr int IPW = (kKT / 4) / SL;  // instructions per wave per tensor
  lds_half *ktile[2], *vtile[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    ktile[b] = tiles + ((size_t)(kg * 2 + b) * 2 + 0) * Lay::kTileHalfs;
    vtile[b] = tiles + ((size_t)(kg * 2 + b) * 2 + 1) * Lay::kTileHalfs;
  }
  int lane_row[IPW], lane_off[IPW];
  unsigned lane_boff[IPW];  // byte offset from the tile's first slot
#pragma unroll
  for (int j = 0; j < IPW; ++j) {
    const int r = 4 * (slab + SL * j) + (lane >> 4);
    lane_row[j] = r;
    lane_off[j] = kvh * HD + 8 * ((lane & 15) ^ swz(r));
    lane_boff[j] = (unsigned)(r * kv_dim + lane_off[j]) * 2u;
  }
  const _Float16 *const kc = p.kc, *const vc = p.vc;
  const _Float16 *const kst = p.kstage, *const vst = p.vstage;
  const int kb0 = ks + kKT * g_first;  // first key of this group's tile 0
#define MIA_LOAD_K(i, buf)                                                                    \
  load_tensor<IPW, SL>(kc, kst, kb0 + kKT * (i), ke, p.start_pos, p.max_seq, kv_dim, lane_row, \
                       lane_off, lane_boff, slab, ktile[buf])
#define MIA_LOAD_V(i, buf)                                                                    \
  load_tensor<IPW, SL>(vc, vst, kb0 + kKT * (i), ke, p.start_pos, p.max_seq, kv_dim, lane_row, \
                       lane_off, lane_boff, slab, vtile[buf])
  // K of tiles 0 and 1 and V of tile 0 go out before the query loads.
  if (g_count > 0) {
    MIA_LOAD_K(0, 0);
    MIA_LOAD_V(0, 0);
  }
  if (g_count > 1) MIA_LOAD_K(1, 1);

  // RoPE (cos, sin) for the workgroup's queries, fl32(theta_inv[i] * pos) as
  // vDSP_vsmul (mistral_model.h:87-88).
  if (p.theta_inv != nullptr) {
    for (int i = tid; i < QT * 64; i += 64 * NW) {
      const int qi = i >> 6, pr = i & 63;
      const int tq = min(tq0 + qi, p.S - 1);
      float ang = p.theta_inv[pr] * (float)(p.start_pos + tq);
      float sn, cs;
      sincosf(ang, &sn, &cs);
      rope[i] = make_float2(cs, sn);
    }
    __syncthreads();
  }

  // Q^T operand: col = row, k-step st covers dims 16*st + 8*half .. +8.
  h8 qb[8];
  {
    const float *qsrc = p.Q + (size_t)(row_valid ? t : 0) * dim_model + (size_t)(kvh * G + g) * HD;
    const float2 *rt = rope + (row_valid ? t - tq0 : 0) * 64;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const f4 *src = reinterpret_cast<const f4 *>(qsrc + 16 * st + 8 * half);
      f4 a = src[0], b = src[1];
      float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      if (p.theta_inv != nullptr) {
#pragma unroll
        for (int pi = 0; pi < 4; ++pi) {
          float2 cs = rt[8 * st + 4 * half + pi];
          rope_pair(v[2 * pi], v[2 * pi + 1], cs.x, cs.y);
        }
      }
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

  // S^T block of one tile: keys x this slab's 32 rows; s[i] is key
  // kb + (i/4)*8 + 4*half + (i%4) for row `row`.
  auto qk = [&](lds_half *kt) {
    f16v s;
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = 0.f;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      h8 a = *(lds_h8 *)(kt + col * HD + 8 * ((2 * st + half) ^ swz(col)));
      s = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, qb[st], s, 0, 0, 0);
    }
    return s;
  };
  // Window mask (only for tiles crossing a window edge of the slab) and the
  // row max over the tile.
  auto mask_max = [&](f16v &s, int kb) {
    const bool inside = slab_full && kb >= lo_max && kb + kKT - 1 <= hi_min && kb + kKT <= ke;
    if (!inside) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kb + (i >> 2) * 8 + 4 * half + (i & 3);
        const bool ok = row_valid && key >= lo_t && key <= hi_t && key < ke;
        s[i] = ok ? s[i] : -INFINITY;
      }
    }
    float m = s[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) m = fmaxf(m, s[i]);
    return fmaxf(m, __shfl_xor(m, 32));
  };

  // Software pipeline over this group's tiles: iteration it holds the masked
  // scores of tile it (s_cur, row max m_cur), computes the scores of tile
  // it+1 on MFMA while the exponentials of tile it are formed, then adds
  // P.V of tile it.  Buffers: K(i) in ktile[i&1], V(i) in vtile[i&1]; during
  // iteration it the loads of K(it+2) and V(it+1) are in flight.
  asm volatile("s_waitcnt vmcnt(0)");
  __syncthreads();
  f16v s_cur = qk(ktile[0]);
  float m_cur = mask_max(s_cur, kb0);

  for (int it = 0; it < n_iter; ++it) {
    // this wave's loads of K(it+1) and V(it) have landed; after the barrier
    // every wave's have, and every wave is done with K(it) and V(it-1)
    asm volatile("s_waitcnt vmcnt(0)");
    __syncthreads();
    if (it + 2 < g_count) MIA_LOAD_K(it + 2, it & 1);
    if (it + 1 < g_count) MIA_LOAD_V(it + 1, (it + 1) & 1);
    if (it < g_count) {
      // Lazy rescale: m_run is the reference max of the row's exponentials
      // and moves only when a score exceeds it by more than 8 (log2 domain),
      // so every p = 2^(s - m_run) stays <= 256 (exact range for fp16) and
      // the accumulators are rescaled rarely.  Normalisation by l at the end
      // is unaffected by the choice of reference.
      const bool move = m_cur > m_run + 8.0f;
      if (__ballot(move) != 0) {  // wave-uniform
        // rows that do not move keep alpha = 1 (also while still fully
        // masked, m_run = -inf); the first move of a row gives alpha = 0
        const float alpha = move ? fast_exp2(m_run - m_cur) : 1.0f;
        const float m_ref = move ? m_cur : m_run;
        l_run *= alpha;
#pragma unroll
        for (int db = 0; db < 4; ++db)
#pragma unroll
          for (int i = 0; i < 16; ++i) o[db][i] *= alpha;
        m_run = m_ref;
      }
      const float m_use = m_run == -INFINITY ? 0.f : m_run;
      // All LDS operands of the iteration are requested up front: K of tile
      // it+1 (stale, unused data when it+1 == g_count) and V^T of tile it.
      lds_half *kt = ktile[(it + 1) & 1];
      lds_half *vt = vtile[it & 1];
      h8 ka[8];
#pragma unroll
      for (int st = 0; st < 8; ++st)
        ka[st] = *(lds_h8 *)(kt + col * HD + 8 * ((2 * st + half) ^ swz(col)));
      // O^T += V^T P^T; k-step kst covers keys 16*kst .. +16, this half's 8
      // keys being {0-3, 8-11} + 4*half (the S^T row permutation).
      h8 va[2][4];
#pragma unroll
      for (int kst = 0; kst < 2; ++kst) {
        const int k0 = 16 * kst + 4 * half;
#pragma unroll
        for (int db = 0; db < 4; ++db) {
          const int d0 = 32 * db + 16 * ((lane >> 4) & 1);
          h4 lo = read_vt4(vt, k0, d0, lane);
          h4 hi = read_vt4(vt, k0 + 8, d0, lane);
          va[kst][db] = h8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
      }
      h8 pb[2];  // P^T B operands for keys 0..15 and 16..31 of the tile
      float lsum = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float pv = fast_exp2(s_cur[i] - m_use);
        lsum += pv;
        pb[i >> 3][i & 7] = (_Float16)pv;
      }
      l_run += lsum;
      f16v s_next;
#pragma unroll
      for (int i = 0; i < 16; ++i) s_next[i] = 0.f;
#pragma unroll
      for (int st = 0; st < 8; ++st)
        s_next = __builtin_amdgcn_mfma_f32_32x32x16_f16(ka[st], qb[st], s_next, 0, 0, 0);
#pragma unroll
      for (int kst = 0; kst < 2; ++kst)
#pragma unroll
        for (int db = 0; db < 4; ++db)
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_f16(va[kst][db], pb[kst], o[db], 0, 0, 0);
      m_cur = mask_max(s_next, kb0 + kKT * (it + 1));
      s_cur = s_next;
    }
  }
#undef MIA_LOAD_K
#undef MIA_LOAD_V
  __syncthreads();  // the merge below reuses the tile area

  // Merge the KH key groups (LDS; the tile area is free after the loop).
  const float l_tot = l_run + __shfl_xor(l_run, 32);
  float *mo = reinterpret_cast<float *>(smem);             // [KH][SL][32][HD]
  float *mml = mo + (size_t)KH * SL * 32 * HD;              // [KH][SL][32][2]
  {
    float *dst = mo + ((size_t)(kg * SL + slab) * 32 + col) * HD;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int i4 = 0; i4 < 4; ++i4)
        *reinterpret_cast<f4 *>(dst + 32 * db + 8 * i4 + 4 * half) =
            f4{o[db][4 * i4 + 0], o[db][4 * i4 + 1], o[db][4 * i4 + 2], o[db][4 * i4 + 3]};
    if (half == 0)
      *reinterpret_cast<float2 *>(mml + ((size_t)(kg * SL + slab) * 32 + col) * 2) =
          make_float2(m_run, l_tot);
  }
  __syncthreads();

  // Thread -> (row, 4 dims) items of the workgroup's RT rows.
  const size_t tile_id = (size_t)kvh * p.n_rtiles + rtile;
  for (int itm = tid; itm < RT * (HD / 4); itm += 64 * NW) {
    const int rl = itm / (HD / 4), d4 = itm % (HD / 4);
    const int sl = rl / 32, rr = rl % 32;
    const int rrow = row0 + rl;
    const int tt = rrow / G, gg = rrow % G;
    if (tt >= p.S) continue;
    float M = -INFINITY;
#pragma unroll
    for (int k = 0; k < KH; ++k) M = fmaxf(M, mml[((size_t)(k * SL + sl) * 32 + rr) * 2]);
    const float Mu = M == -INFINITY ? 0.f : M;
    float Ls = 0.f;
    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < KH; ++k) {
      const size_t r = (size_t)(k * SL + sl) * 32 + rr;
      const float2 ml = *reinterpret_cast<const float2 *>(mml + r * 2);
      const float e = fast_exp2(ml.x - Mu);
      Ls = __builtin_fmaf(e, ml.y, Ls);
      acc += e * *reinterpret_cast<const f4 *>(mo + r * HD + 4 * d4);
    }
    if (p.nsplit == 1) {
      *reinterpret_cast<f4 *>(p.out + (size_t)tt * dim_model + (size_t)(kvh * G + gg) * HD +
                              4 * d4) = acc * (1.0f / Ls);
    } else {
      const size_t pidx = (tile_id * p.nsplit + split) * RT + rl;
      *reinterpret_cast<f4 *>(p.part_o + pidx * HD + 4 * d4) = acc;
      if (d4 == 0) *reinterpret_cast<float2 *>(p.part_ml + pidx * 2) = make_float2(M, Ls);
    }
  }
}

// Split merge: one workgroup per 8 rows of a tile, thread = (row, 4 dims).  A
// separate launch, so the kernel boundary orders the partial writes before
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
  const float Mu = M == -INFINITY ? 0.f : M;
  float Ls = 0.f;
  f4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int sp = 0; sp < p.nsplit; ++sp) {
    const size_t idx = ((size_t)tile_id * p.nsplit + sp) * rt + rl;
    float2 ml = *reinterpret_cast<const float2 *>(p.part_ml + idx * 2);
    float e = fast_exp2(ml.x - Mu);
    Ls = __builtin_fmaf(e, ml.y, Ls);
    acc += e * *reinterpret_cast<const f4 *>(p.part_o + idx * HD + 4 * d4);
  }
  *reinterpret_cast<f4 *>(p.out + (size_t)t * dim_model + (size_t)(kvh * G + g) * HD + 4 * d4) =
      acc * (1.0f / Ls);
}

template <int SL, int KH>
hipError_t launch_variant(const FlashParams &p, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  using Lay = FlashLayout<SL, KH>;
  static bool attr_set = false;
  if (!attr_set) {
    hipError_t e = hipFuncSetAttribute((const void *)flash_kernel<4, SL, KH>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)Lay::kBytes);
    if (e != hipSuccess) return e;
    attr_set = true;
  }
  dim3 grid(p.n_kv * p.n_rtiles * p.nsplit);
  hipExtLaunchKernelGGL((flash_kernel<4, SL, KH>), grid, dim3(64 * SL * KH), Lay::kBytes, s, ev0, ev1,
                        0, p);
  return hipGetLastError();
}

}  // namespace

size_t flash_scratch_bytes(int n_kv, int n_rtiles, int nsplit, int rows_per_tile) {
  return (size_t)n_kv * n_rtiles * nsplit * rows_per_tile * (HD + 2) * sizeof(float);
}

// Few rows (S*G <= 32, e.g. speculative verify): one slab, 4 key groups, and
// key splits over workgroups until about target_wgs workgroups.  Otherwise
// (prefill): two slabs (64 rows) and 4 key groups per workgroup, no split
// unless the row tiles alone leave the device mostly idle.
void flash_plan(int S, int n_kv, int G, int start_pos, int max_seq, int target_wgs, int *n_rtiles,
                int *nsplit, int *split_keys, int *rows_per_tile) {
  const int rows = S * G;
  const int rt = rows <= 32 ? 32 : 64;
  const int ntiles = (rows + rt - 1) / rt;
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
  long want = (long)target_wgs / ((long)n_kv * ntiles);
  if (want < 1) want = 1;
  // at least 4 tiles of 32 keys per key group and split
  long max_split = maxkeys / (4L * 4 * kKT);
  if (want > max_split) want = max_split > 0 ? max_split : 1;
  long sk = (maxkeys + want - 1) / want;
  sk = ((sk + kKT - 1) / kKT) * kKT;
  long ns = (maxkeys + sk - 1) / sk;
  if (ns < 1) ns = 1;
  *n_rtiles = ntiles;
  *nsplit = (int)ns;
  *split_keys = (int)sk;
  *rows_per_tile = rt;
}

hipError_t launch_flash(const FlashParams &p, int G, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  if (G != 4) return hipErrorInvalidValue;
  const int rt = p.S * G <= 32 ? 32 : 64;
  return rt == 32 ? launch_variant<1, 4>(p, s, ev0, ev1) : launch_variant<2, 4>(p, s, ev0, ev1);
}

hipError_t launch_flash_merge(const FlashParams &p, hipStream_t s) {
  const int rt = p.S * 4 <= 32 ? 32 : 64;
  if (p.nsplit > 1)
    hipLaunchKernelGGL((flash_merge_kernel<4>), dim3(p.n_kv * p.n_rtiles * (rt / 8)), dim3(256), 0,
                       s, p, rt);
  return hipGetLastError();
}

}  // namespace mia
