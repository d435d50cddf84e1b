// mia_decode.hip -- S=1 GQA decode attention for gfx950 (split-K flash-decode).
//
// Replaces mistral/mistral_model.h:362-487 (gqa_attention_neon), and, in the
// fused variant, steps 4-6 of mistral/mistral_model.h:849-863 (RoPE on q/k,
// fp16 round of k/v, ring write at pos % max_seq, attention).
//
// Grid: one workgroup per (kv head, chunk of the window), 8 waves per
// workgroup, all on that head.  Chunk c is the 16-key tiles c, c + nchunk,
// c + 2 nchunk, ... of the window: spread over the whole ring rather than one
// contiguous block, every workgroup draws on all memory channels alike; wave
// w of the workgroup takes every 8th of its chunk's tiles.  The heads of one
// chunk are consecutive workgroups, which the dispatcher spreads over the
// XCDs.  32 chunks at 8 kv heads fill 256 CUs with 8x fewer split-K partials
// than one wave per head and chunk would leave.
//
// Each wave is an independent pipeline over its tiles, held in a ring of
// register buffers so that the next tiles' loads are in flight while one
// tile is computed.  Every load instruction reads 4 rows x 256 B (whole
// 128-byte lines; loads of 16 rows x 64 B each read a measured 6 % slower):
//   scores  v_mfma_f32_16x16x32_f16: A = 16 key rows (lane = key row), from
//           the loaded K rows re-laid through a per-wave LDS tile; B = the
//           G=4 query heads of the group with q split into fp16 hi + lo
//           parts along K (q = hi + lo to ~2^-22), so the scores carry fp32 q
//           accuracy.
//   softmax wave-local online max / sum in the log2 domain.
//   P.V     v_mfma_f32_16x16x16_f16 computing O^T = V^T P^T: the score
//           accumulator layout (lane = 4 keys of one head) is already the B
//           operand layout with keys along K, so P (fp16 hi + lo) never
//           leaves its lane; V^T comes from the 4 loaded V rows of the lane
//           (4 keys x 8 dims) by byte permutes.
// The 8 waves' results merge through LDS into the chunk's partial (m, l, o)
// (the final output when there is one chunk); a second, small kernel does
// the log-sum-exp merge over chunks.
#include <type_traits>

#include "mia_device.h"
#include "mia_kernels.h"

namespace mia {

namespace {

constexpr int kWaves = 8;         // waves per workgroup, all on one kv head
constexpr int kThreads = 64 * kWaves;
constexpr int kTile = 16;        // keys per wave tile
// Register tile buffers per wave.  One: the buffer is refilled while it is
// consumed (K once staged to LDS, V after the P.V MFMAs), so one tile per wave
// is in flight while the current one is processed.  Two buffers kept more
// loads in flight and read the window ~4 % slower.
constexpr int kDepth = 1;
constexpr int kMaxChunks = 256;  // merge capacity per kv head
constexpr int G = 4;             // query heads per kv head
// Bytes per staged K row: 16 B of padding put the 16 rows of a column read
// on 16 different bank groups.
constexpr int kKPitch = HD * 2 + 16;
static_assert(kThreads == G * HD, "the in-workgroup merge gives each thread one output element");

struct DecodeSmem {
  float2 cs[kWaves][64];                  // per-wave RoPE (cos, sin) of the 64 pair indices
  unsigned char kst[kWaves][kTile * kKPitch];  // per-wave K tile in row-major order
  _Float16 knew[HD];                      // rotated fp16 new key (the wave that attends it)
  _Float16 vnew[HD];
  float mo[kWaves][G][HD];                // in-workgroup merge: each wave's o
  float2 mlw[kWaves][G];                  // ... and its (m, l)
};

struct TileBuf {
  u4 k[4];  // K rows 4*(lane/16) + m, dims 8*(lane%16) .. +8
  u4 v[4];  // V rows 4*(lane/16) + m, dims 8*(lane%16) .. +8
};

// Value of x in lane `src` (uniform result).
__device__ __forceinline__ float lane_value(float x, int src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), src));
}

__device__ __forceinline__ int ring_slot(int start, int t, int max_seq) {
  int s = start + t;
  return s >= max_seq ? s - max_seq : s;
}

// kPlain: q already rotated, one token at p.pos.  kFused: the decode step
// (RoPE of q and k at p.pos, the new token's write, attention).  kPositions:
// token blockIdx.y at p.positions[blockIdx.y] over the ring as it stands
// (the chunked prefill's phase 2), q rotated in-kernel when theta_inv is set.
enum { kPlain = 0, kFused = 1, kPositions = 2 };

template <int MODE>
__global__ void __launch_bounds__(kThreads, 1) decode_kernel(DecodeParams p) {
  __shared__ DecodeSmem sm;
  constexpr bool FUSED = MODE == kFused;

  // This workgroup's token: window, query, output and partial rows.
  int pos = p.pos, win_L = p.L, win_start = p.start;
  const float *q_in = p.q;
  float *out = p.out, *part_o = p.part_o, *part_ml = p.part_ml;
  if (MODE == kPositions) {
    const int tok = blockIdx.y;
    pos = p.positions[tok];
    // mistral_model.h:964-967; a negative position has an empty window
    // (pos + 1 is not formed: it would overflow at INT_MAX)
    win_L = pos < 0 ? 0 : (pos < p.max_seq - 1 ? pos + 1 : p.max_seq);
    win_start = pos < 0 ? 0 : (int)(((long)pos + 1 - win_L) % p.max_seq);
    const size_t rows = (size_t)p.n_kv * G;  // query heads
    q_in += (size_t)tok * rows * HD;
    out += (size_t)tok * rows * HD;
    part_o += (size_t)tok * rows * p.nchunk * HD;
    part_ml += (size_t)tok * rows * p.nchunk * 2;
  }
  const bool rope_q = FUSED || (MODE == kPositions && p.theta_inv != nullptr);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lc = lane & 15;  // MFMA column / V dim block
  const int lg = lane >> 4;  // MFMA k group / V key group
  const int kvh = blockIdx.x % p.n_kv;
  const int chunk = blockIdx.x / p.n_kv;
  const int kv_dim = p.n_kv * HD;
  // The new token (fused) is attended after the loop, from its fp16 copy in
  // LDS, by the last wave of the last chunk; the tiles cover keys [0, ce).
  const int ce = FUSED ? win_L - 1 : win_L;
  const int n_tiles = (ce + kTile - 1) / kTile;
  const bool has_new = FUSED && chunk == p.nchunk - 1 && w == kWaves - 1;
  // Tiles of this wave: chunk + nchunk * (w + kWaves * i), i = 0, 1, ...
  const int t_first = chunk + p.nchunk * w, t_step = p.nchunk * kWaves;
  int s_next = 0;
  const int s_end = t_first < n_tiles ? (n_tiles - 1 - t_first) / t_step + 1 : 0;
  auto next_tile = [&]() -> int { return s_next < s_end ? t_first + t_step * s_next++ : -1; };

  const _Float16 *kbase = p.kc + (size_t)kvh * HD;
  const _Float16 *vbase = p.vc + (size_t)kvh * HD;

  // Tile loads: lane (lc, lg) reads rows 4*lg + m, dims 8*lc .. +8 of K and
  // of V.  A tile whose 16 slots are contiguous in the ring and inside the
  // window (all but the tile across the ring's end and the window's last
  // tile) is addressed as one wave-uniform row base plus fixed per-lane
  // offsets; the others clamp and wrap per lane.
  unsigned roff[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) roff[m] = (unsigned)(4 * lg + m) * kv_dim + 8 * lc;
  auto tile_row0 = [&](int tt, bool &linear) {
    const int t0 = tt * kTile;
    const int s0 = ring_slot(win_start, t0, p.max_seq);
    linear = s0 + kTile <= p.max_seq && t0 + kTile <= ce;
    return t0;
  };
  // Every refill issues its loads, also past the end of the wave's tiles
  // (tt < 0: all lanes read one 16-byte piece, a cache hit): with the same
  // number of loads on every path the compiler can wait for exactly the
  // buffer it needs instead of for all outstanding loads.
  // (Offsets rather than pointers are selected, so that every load keeps
  // the global address space of the kernel argument.)
  // (In-layer offsets reach max_seq * kv_dim elements, beyond 32 bits for
  // large rings: the per-lane slot offsets are formed in 64 bits.)
  auto issue_rows = [&](u4 (&dst)[4], const _Float16 *base, int tt) {
    size_t row0 = 0;
    size_t off[4] = {0, 0, 0, 0};
    if (tt >= 0) {
      bool linear;
      const int t0 = tile_row0(tt, linear);
      if (linear) {
        row0 = (size_t)ring_slot(win_start, t0, p.max_seq) * kv_dim;
#pragma unroll
        for (int m = 0; m < 4; ++m) off[m] = roff[m];
      } else {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int t = min(t0 + 4 * lg + m, ce - 1);
          off[m] = (size_t)ring_slot(win_start, t, p.max_seq) * kv_dim + 8 * lc;
        }
      }
    }
    const _Float16 *src = base + row0;
#pragma unroll
    for (int m = 0; m < 4; ++m) dst[m] = *reinterpret_cast<const u4 *>(src + off[m]);
  };
  auto issue_k = [&](TileBuf &b, int tt) { issue_rows(b.k, kbase, tt); };
  auto issue_v = [&](TileBuf &b, int tt) { issue_rows(b.v, vbase, tt); };
  auto issue = [&](TileBuf &b, int tt) {
    issue_k(b, tt);
    issue_v(b, tt);
  };

  // The prologue's own loads (q, theta_inv, the new token) are issued before
  // the first kDepth tiles: loads complete in issue order, so the q set-up
  // waits only for its own data, not for the tiles.
  const bool col = lc < G;
  f4 qraw[8];
  {
    const f4 *qsrc = reinterpret_cast<const f4 *>(q_in + (size_t)(kvh * G + (col ? lc : 0)) * HD + 8 * lg);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      qraw[2 * s] = qsrc[8 * s];
      qraw[2 * s + 1] = qsrc[8 * s + 1];
    }
  }
  const float th_in = rope_q ? p.theta_inv[lane] : 0.f;
  float2 knew_in = make_float2(0.f, 0.f), vnew_in = make_float2(0.f, 0.f);
  if (FUSED) {  // (every wave: a branch here would make the join wait for the loads)
    knew_in = *reinterpret_cast<const float2 *>(p.knew + (size_t)kvh * HD + 2 * lane);
    vnew_in = *reinterpret_cast<const float2 *>(p.vnew + (size_t)kvh * HD + 2 * lane);
  }

  TileBuf buf[kDepth];
  int tix[kDepth];
#pragma unroll
  for (int b = 0; b < kDepth; ++b) {
    tix[b] = next_tile();
    issue(buf[b], tix[b]);
  }
  // (keeps the compiler from converting the new token before the tile loads
  // are issued, which would wait for its loads there)
  if (FUSED) asm volatile("" : "+v"(knew_in.x), "+v"(knew_in.y), "+v"(vnew_in.x), "+v"(vnew_in.y));

  float2 cs_lane = make_float2(1.f, 0.f);  // (cos, sin) of pair `lane`
  if (rope_q) {
    // angle = fl32(theta_inv[i] * pos) as vDSP_vsmul (mistral_model.h:87-88)
    const float ang = th_in * (float)pos;
    float sn, cs;
    sincosf(ang, &sn, &cs);
    cs_lane = make_float2(cs, sn);
    sm.cs[w][lane] = cs_lane;
    wave_lds_sync();
  }
  if (has_new) {
    // new k rotated (pair `lane`) and v, rounded to fp16 (mistral_model.h:854-857)
    float2 kv = knew_in;
    rope_pair(kv.x, kv.y, cs_lane.x, cs_lane.y);
    const float2 vv = vnew_in;
    sm.knew[2 * lane] = (_Float16)kv.x;
    sm.knew[2 * lane + 1] = (_Float16)kv.y;
    sm.vnew[2 * lane] = (_Float16)vv.x;
    sm.vnew[2 * lane + 1] = (_Float16)vv.y;
    wave_lds_sync();
    if (lane < 16) {  // write of the new row (256 B per tensor)
      const size_t row = p.new_k ? 0 : (size_t)p.new_slot * kv_dim;
      _Float16 *kd = (p.new_k ? p.new_k : p.kc) + row, *vd = (p.new_v ? p.new_v : p.vc) + row;
      const size_t off = (size_t)kvh * HD + 8 * lane;
      *reinterpret_cast<u4 *>(kd + off) = *reinterpret_cast<const u4 *>(&sm.knew[8 * lane]);
      *reinterpret_cast<u4 *>(vd + off) = *reinterpret_cast<const u4 *>(&sm.vnew[8 * lane]);
    }
  }

  // B operand: column lc < G is query head kvh*G + lc; k-step s covers dims
  // 32*s + 8*lg .. +8 (the same dims the A lanes load), hi and lo parts.
  h8 qhi[4], qlo[4];
  {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const f4 a = qraw[2 * s], b = qraw[2 * s + 1];
      float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      if (rope_q) {
#pragma unroll
        for (int pi = 0; pi < 4; ++pi) {
          float2 cs = sm.cs[w][16 * s + 4 * lg + pi];
          rope_pair(v[2 * pi], v[2 * pi + 1], cs.x, cs.y);
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float x = col ? v[e] * p.qscale : 0.f;
        _Float16 hi = (_Float16)x;
        qhi[s][e] = hi;
        qlo[s][e] = (_Float16)(x - (float)hi);
      }
    }
  }


  // m_run[g]: wave-uniform running max of head g; m_lane: the same value for
  // the head of this lane's MFMA column (lanes with lc >= G carry junk).
  // o[e]: O^T accumulator of MFMA e (dims 8*(4*lg+i) + e, head lc).
  float m_run[G], m_lane = -INFINITY, l_part = 0.f;
  f4 o[8];
#pragma unroll
  for (int g = 0; g < G; ++g) m_run[g] = -INFINITY;
#pragma unroll
  for (int e = 0; e < 8; ++e) o[e] = f4{0.f, 0.f, 0.f, 0.f};

  // One 16-key tile starting at key t0; keys >= cend are masked.  With
  // `refill` the buffer is refilled with tile `next`: its K half as soon as
  // the K rows are in LDS, its V half after the P.V MFMAs.
  unsigned char *kst = sm.kst[w];
  auto process = [&](TileBuf &b, int t0, int cend, int next, auto refill) {
    // K rows -> LDS (row-major) -> A operand of k-step s: key row lc, dims
    // 32*s + 8*lg .. +8.
    wave_lds_sync();  // (the previous tile's reads of kst come first)
#pragma unroll
    for (int m = 0; m < 4; ++m)
      *reinterpret_cast<u4 *>(kst + (4 * lg + m) * kKPitch + 16 * lc) = b.k[m];
    wave_lds_sync();
    if (refill) issue_k(b, next);
    h8 ka[4];
#pragma unroll
    for (int s = 0; s < 4; ++s)
      ka[s] = *reinterpret_cast<const h8 *>(kst + lc * kKPitch + 64 * s + 16 * lg);
    f4 d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[s], qhi[s], d, 0, 0, 0);
      d = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka[s], qlo[s], d, 0, 0, 0);
    }
    // d[i]: score of key t0 + 4*lg + i for head lc (lanes lc < G).
    float sc[4];
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      sc[i] = (t0 + 4 * lg + i < cend) ? d[i] : -INFINITY;
      mx = fmaxf(mx, sc[i]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    // every lane of column lc now holds the tile max of head lc
    const float m_lane_new = fmaxf(m_lane, mx);
    bool grow = false;
#pragma unroll
    for (int g = 0; g < G; ++g) grow |= lane_value(m_lane_new, g) > m_run[g];
    if (grow) {  // wave-uniform
      const float alpha = fast_exp2(m_lane - m_lane_new);  // per column (head)
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] *= alpha;
      l_part *= alpha;
#pragma unroll
      for (int g = 0; g < G; ++g) m_run[g] = lane_value(m_lane_new, g);
    }
    m_lane = m_lane_new;
    // P^T as the B operand of O^T += V^T P^T (k = this lane group's 4 keys,
    // column = head lc), split into fp16 hi + lo parts.
    h4 phi, plo;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float pv = lc < G ? fast_exp2(sc[i] - m_lane) : 0.f;
      l_part += pv;
      _Float16 h = (_Float16)pv;
      phi[i] = h;
      plo[i] = (_Float16)(pv - (float)h);
    }
    // A operand of MFMA e: V^T rows = dims 8*lc + e, k = keys 4*lg + m, i.e.
    // element e of the 4 loaded V rows, gathered with byte permutes.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const unsigned a0 = b.v[0][j], a1 = b.v[1][j], a2 = b.v[2][j], a3 = b.v[3][j];
      u2 lo = {__builtin_amdgcn_perm(a1, a0, 0x05040100u), __builtin_amdgcn_perm(a3, a2, 0x05040100u)};
      u2 hi = {__builtin_amdgcn_perm(a1, a0, 0x07060302u), __builtin_amdgcn_perm(a3, a2, 0x07060302u)};
      const h4 ae = __builtin_bit_cast(h4, lo), ao = __builtin_bit_cast(h4, hi);
      o[2 * j] = __builtin_amdgcn_mfma_f32_16x16x16f16(ae, phi, o[2 * j], 0, 0, 0);
      o[2 * j] = __builtin_amdgcn_mfma_f32_16x16x16f16(ae, plo, o[2 * j], 0, 0, 0);
      o[2 * j + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(ao, phi, o[2 * j + 1], 0, 0, 0);
      o[2 * j + 1] = __builtin_amdgcn_mfma_f32_16x16x16f16(ao, plo, o[2 * j + 1], 0, 0, 0);
    }
    if (refill) issue_v(b, next);
  };

  // Ring of kDepth register buffers: buffer b is refilled with the next tile
  // of the stream while it is consumed (K once staged, V after the P.V
  // MFMAs).
  // Tiles come in stream order, so the first empty buffer ends the loop.
  for (bool more = tix[0] >= 0; more;) {
#pragma unroll
    for (int b = 0; b < kDepth; ++b) {
      if (tix[b] < 0) {
        more = false;
        break;
      }
      const int nt = next_tile();
      process(buf[b], tix[b] * kTile, ce, nt, std::true_type{});
      tix[b] = nt;
    }
  }
  if (has_new) {
    // Every row of this tile is the new key / value; only key 0 is unmasked.
    TileBuf nb;
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      nb.k[m] = *reinterpret_cast<const u4 *>(&sm.knew[8 * lc]);
      nb.v[m] = *reinterpret_cast<const u4 *>(&sm.vnew[8 * lc]);
    }
    process(nb, win_L - 1, win_L, -1, std::false_type{});
  }

  // Wave totals: l over the 4 key groups of column lc.
  l_part += __shfl_xor(l_part, 16);
  l_part += __shfl_xor(l_part, 32);
  // The waves' (m, l, o) into LDS: lane (lc, lg) holds dims 32*lg .. +32 of
  // head lc, element i of o[e] being dim 8*(4*lg + i) + e.
  if (lc < G) {
    float *mo = sm.mo[w][lc] + 32 * lg;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<f4 *>(mo + 8 * i) = f4{o[0][i], o[1][i], o[2][i], o[3][i]};
      *reinterpret_cast<f4 *>(mo + 8 * i + 4) = f4{o[4][i], o[5][i], o[6][i], o[7][i]};
    }
    if (lg == 0) sm.mlw[w][lc] = make_float2(m_lane, l_part);
  }
  __syncthreads();
  // Thread (g, d) merges element d of head g over the waves (a wave without
  // keys has m = -inf, l = 0).
  const int g = tid / HD, d = tid % HD;
  float M = -INFINITY;
#pragma unroll
  for (int v = 0; v < kWaves; ++v) M = fmaxf(M, sm.mlw[v][g].x);
  float L = 0.f, O = 0.f;
#pragma unroll
  for (int v = 0; v < kWaves; ++v) {
    const float2 ml = sm.mlw[v][g];
    const float e = ml.x == -INFINITY ? 0.f : fast_exp2(ml.x - M);
    L = __builtin_fmaf(e, ml.y, L);
    O = __builtin_fmaf(e, sm.mo[v][g][d], O);
  }
  if (p.nchunk == 1) {
    // (an empty window, only in kPositions, writes zeros)
    out[((size_t)kvh * G + g) * HD + d] = L > 0.f ? O / L : 0.f;
  } else {
    const size_t row = ((size_t)kvh * p.nchunk + chunk) * G + g;
    part_o[row * HD + d] = O;
    if (d == 0) *reinterpret_cast<float2 *>(part_ml + row * 2) = make_float2(M, L);
  }
}

// Cross-chunk log-sum-exp merge.  Workgroup = (kv head, q head, block of
// kMergeDims dims); thread = (chunk group cg, dim d).  Every load (the chunk
// maxima and sums, and the thread's partial outputs) is issued before the
// first reduction, so the merge costs one memory round trip.  A separate
// launch: the kernel boundary orders the partial writes before these reads.
// 16 dims per workgroup (256 workgroups for 8 kv heads) measured 1.6 %
// faster per decode step than 32 (128 workgroups) and than 8 (512).
constexpr int kMergeDims = 16;

__global__ void __launch_bounds__(256) decode_merge_kernel(DecodeParams p) {
  constexpr int kDW = kMergeDims;      // dims of one workgroup
  constexpr int kCG = 256 / kDW;       // chunk groups (threads per dim)
  constexpr int kPer = kMaxChunks / kCG;  // chunks per thread at most
  __shared__ float mx[8];
  __shared__ float red[kCG][kDW];
  __shared__ float wt[kMaxChunks];
  __shared__ float lsum[8];
  const int db = blockIdx.x % (HD / kDW);
  const int hg = blockIdx.x / (HD / kDW);  // kvh * G + g
  const int kvh = hg / G, g = hg % G;
  const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
  const int cg = tid / kDW, d = kDW * db + (tid % kDW);
  // token blockIdx.y (kPositions; 0 otherwise): its partials and output rows
  const size_t tok = blockIdx.y;
  const size_t hb = (size_t)kvh * p.nchunk * G + tok * p.n_kv * p.nchunk * G;
  float2 ml = make_float2(-INFINITY, 0.f);
  if (tid < p.nchunk) ml = *reinterpret_cast<const float2 *>(p.part_ml + (hb + (size_t)tid * G + g) * 2);
  float ov[kPer];
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int c = cg + kCG * k;
    ov[k] = c < p.nchunk ? p.part_o[(hb + (size_t)c * G + g) * HD + d] : 0.f;
  }
  // max over chunks
  float m = wave_max(ml.x);
  if (lane == 0) mx[wv] = m;
  __syncthreads();
  float M = mx[0];
#pragma unroll
  for (int k = 1; k < 4; ++k) M = fmaxf(M, mx[k]);
  const float Mu = M == -INFINITY ? 0.f : M;
  const float e = ml.x == -INFINITY ? 0.f : fast_exp2(ml.x - Mu);
  if (tid < kMaxChunks) wt[tid] = e;
  float l = wave_sum(e * ml.y);
  if (lane == 0) lsum[wv] = l;
  __syncthreads();
  float O = 0.f;
#pragma unroll
  for (int k = 0; k < kPer; ++k) {
    const int c = cg + kCG * k;
    if (c < p.nchunk) O = __builtin_fmaf(wt[c], ov[k], O);
  }
  red[cg][tid % kDW] = O;
  __syncthreads();
  if (tid < kDW) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < kCG; ++k) t += red[k][tid];
    const float Ls = lsum[0] + lsum[1] + lsum[2] + lsum[3];
    // (Ls = 0 only for an empty window: zeros)
    p.out[(tok * p.n_kv * G + hg) * HD + d] = Ls > 0.f ? t / Ls : 0.f;
  }
}

}  // namespace

size_t decode_scratch_bytes(int n_kv, int g, int nchunk, int n_tok) {
  return (size_t)n_tok * n_kv * nchunk * g * (HD + 2) * sizeof(float);
}

int decode_pick_nchunk(int L, int n_kv, int target_wgs) {
  const int n_tiles = (L + kTile - 1) / kTile;
  // one workgroup per (kv head, chunk), about target_wgs of them; at least
  // one tile per wave, at most kMaxChunks chunks
  int nchunk = (target_wgs + n_kv - 1) / n_kv;
  const int per_wave = (n_tiles + kWaves - 1) / kWaves;
  if (nchunk > per_wave) nchunk = per_wave;
  if (nchunk > kMaxChunks) nchunk = kMaxChunks;
  if (nchunk < 1) nchunk = 1;
  return nchunk;
}

hipError_t launch_decode(const DecodeParams &p, int g, int mode, hipStream_t s, hipEvent_t ev0,
                         hipEvent_t ev1) {
  if (g != G) return hipErrorInvalidValue;
  if (p.nchunk < 1 || p.nchunk > kMaxChunks) return hipErrorInvalidValue;
  const bool positions = mode == kDecodePositions;
  if (positions && (p.positions == nullptr || p.n_tok < 1 || p.n_tok > 65535))
    return hipErrorInvalidValue;
  dim3 grid(p.n_kv * p.nchunk, positions ? p.n_tok : 1), block(kThreads);
  if (mode == kDecodeFused)
    hipExtLaunchKernelGGL(decode_kernel<kFused>, grid, block, 0, s, ev0, ev1, 0, p);
  else if (positions)
    hipExtLaunchKernelGGL(decode_kernel<kPositions>, grid, block, 0, s, ev0, ev1, 0, p);
  else
    hipExtLaunchKernelGGL(decode_kernel<kPlain>, grid, block, 0, s, ev0, ev1, 0, p);
  return hipGetLastError();
}

hipError_t launch_decode_merge(const DecodeParams &p, hipStream_t s) {
  const int ntok = p.positions != nullptr ? p.n_tok : 1;
  if (p.nchunk > 1)
    hipLaunchKernelGGL(decode_merge_kernel, dim3(p.n_kv * G * (HD / kMergeDims), ntok), dim3(256),
                       0, s, p);
  return hipGetLastError();
}

}  // namespace mia
