// mia_decode.hip -- S=1 GQA decode attention for gfx950 (split-K flash-decode).
//
// Replaces mistral/mistral_model.h:362-487 (gqa_attention_neon), and, in the
// fused variant, steps 4-6 of mistral/mistral_model.h:849-863 (RoPE on q/k,
// fp16 round of k/v, ring write at pos % max_seq, attention).
//
// Grid: one workgroup per (kv head, chunk of the window); blockIdx % n_kv is
// the kv head, so with the hardware's round-robin workgroup dispatch over the
// 8 XCDs every chunk of one kv head (and its partials) stays on one XCD.
//
// Each of the 4 waves of a workgroup is an independent pipeline over 16-key
// tiles (wave w takes tiles w, w+4, ...), held in a ring of register buffers
// so that the next tiles' loads are in flight while one tile is computed:
//   scores  v_mfma_f32_16x16x32_f16: A = 16 key rows straight from the
//           loads (lane = key row, 64 contiguous bytes), B = the G=4 query
//           heads of the group with q split into fp16 hi + lo parts along K
//           (q = hi + lo to ~2^-22), so the scores carry fp32 q accuracy.
//   softmax wave-local online max / sum in the log2 domain.
//   P.V     v_mfma_f32_16x16x16_f16 computing O^T = V^T P^T: the score
//           accumulator layout (lane = 4 keys of one head) is already the B
//           operand layout with keys along K, so P (fp16 hi + lo) never
//           leaves its lane; V^T comes from the 4 loaded V rows of the lane
//           (4 keys x 8 dims) by byte permutes.
// The 4 wave partials are merged in LDS; chunk partials are merged by a
// second, small kernel (log-sum-exp merge).
#include "mia_device.h"
#include "mia_kernels.h"

namespace mia {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = 4;
constexpr int kTile = 16;        // keys per wave tile
constexpr int kDepth = 2;        // register tile buffers per wave (3, 4 measured no faster)
constexpr int kMaxChunks = 256;  // merge capacity per kv head
constexpr int G = 4;             // query heads per kv head

struct DecodeSmem {
  float2 cs[64];                 // RoPE (cos, sin) for the 64 pair indices
  _Float16 knew[HD];             // rotated fp16 new key of this kv head
  _Float16 vnew[HD];
  float ml[kWaves][2 * G];       // per-wave (max, sum)
  float acc[kWaves][G][HD];      // per-wave partial outputs
};

struct TileBuf {
  u4 k[4];  // MFMA A operand, k-step s: key row lane%16, dims 32*s + 8*(lane/16) .. +8
  u4 v[4];  // V rows: keys 4*(lane/16) + m, dims 8*(lane%16) .. +8
};

// Value of x in lane `src` (uniform result).
__device__ __forceinline__ float lane_value(float x, int src) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), src));
}

__device__ __forceinline__ int ring_slot(int start, int t, int max_seq) {
  int s = start + t;
  return s >= max_seq ? s - max_seq : s;
}

template <bool FUSED>
__global__ void __launch_bounds__(kThreads, 3) decode_kernel(DecodeParams p) {
  __shared__ DecodeSmem sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int lc = lane & 15;  // MFMA column / V dim block
  const int lg = lane >> 4;  // MFMA k group / V key group
  const int kvh = blockIdx.x % p.n_kv;
  const int chunk = blockIdx.x / p.n_kv;
  const int kv_dim = p.n_kv * HD;
  // Chunk = tiles [chunk*T/nchunk, (chunk+1)*T/nchunk) of the T 16-key tiles
  // of the window, so workgroups differ by at most one tile.
  const long n_tiles = (p.L + kTile - 1) / kTile;
  const int c0 = (int)((long)chunk * n_tiles / p.nchunk) * kTile;
  const int c1 = min((int)((long)(chunk + 1) * n_tiles / p.nchunk) * kTile, p.L);
  const bool has_new = FUSED && (c1 == p.L);

  // The new token (fused, last chunk) is attended after the loop from its
  // fp16 copy in LDS, so the tiles cover [c0, ce).
  const int ce = has_new ? p.L - 1 : c1;
  // Tiles of this wave: global tile index tt = (c0/16) + w + 4*i.
  const int first_tile = c0 / kTile + w;
  const int end_tile = (ce + kTile - 1) / kTile;  // exclusive
  const int n_my = first_tile < end_tile ? (end_tile - first_tile + kWaves - 1) / kWaves : 0;
  const int last_tile = first_tile + kWaves * (n_my > 0 ? n_my - 1 : 0);

  const _Float16 *kbase = p.kc + (size_t)kvh * HD;
  const _Float16 *vbase = p.vc + (size_t)kvh * HD;

  auto issue = [&](TileBuf &b, int i) {
    const int tt = min(first_tile + kWaves * i, last_tile);  // clamp: re-read, L2 hit
    const int t0 = tt * kTile;
    {
      int t = min(t0 + lc, ce - 1);
      unsigned off = (unsigned)ring_slot(p.start, t, p.max_seq) * (unsigned)kv_dim + 8 * lg;
      const _Float16 *src = kbase + off;
#pragma unroll
      for (int s = 0; s < 4; ++s) b.k[s] = *reinterpret_cast<const u4 *>(src + 32 * s);
    }
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      int t = min(t0 + 4 * lg + m, ce - 1);
      unsigned off = (unsigned)ring_slot(p.start, t, p.max_seq) * (unsigned)kv_dim + 8 * lc;
      b.v[m] = *reinterpret_cast<const u4 *>(vbase + off);
    }
  };

  // The first kDepth tiles are requested before the prologue so that their
  // latency overlaps the RoPE table, the new-token write and the q set-up.
  TileBuf buf[kDepth];
  if (n_my > 0) {
#pragma unroll
    for (int b = 0; b < kDepth; ++b) issue(buf[b], b);
  }

  if (FUSED) {
    if (tid < 64) {
      // angle = fl32(theta_inv[i] * pos) as vDSP_vsmul (mistral_model.h:87-88)
      float ang = p.theta_inv[tid] * (float)p.pos;
      float sn, cs;
      sincosf(ang, &sn, &cs);
      sm.cs[tid] = make_float2(cs, sn);
    }
    __syncthreads();
    if (has_new && tid < 64) {
      // new k rotated (pair tid) and v, rounded to fp16 (mistral_model.h:854-857)
      float2 kv = *reinterpret_cast<const float2 *>(p.knew + (size_t)kvh * HD + 2 * tid);
      float2 cs = sm.cs[tid];
      rope_pair(kv.x, kv.y, cs.x, cs.y);
      float2 vv = *reinterpret_cast<const float2 *>(p.vnew + (size_t)kvh * HD + 2 * tid);
      sm.knew[2 * tid] = (_Float16)kv.x;
      sm.knew[2 * tid + 1] = (_Float16)kv.y;
      sm.vnew[2 * tid] = (_Float16)vv.x;
      sm.vnew[2 * tid + 1] = (_Float16)vv.y;
    }
    __syncthreads();
    if (has_new && tid < 16) {  // ring write of the new row (256 B per tensor)
      size_t off = (size_t)p.new_slot * kv_dim + (size_t)kvh * HD + 8 * tid;
      *reinterpret_cast<u4 *>(p.kc + off) = *reinterpret_cast<const u4 *>(&sm.knew[8 * tid]);
      *reinterpret_cast<u4 *>(p.vc + off) = *reinterpret_cast<const u4 *>(&sm.vnew[8 * tid]);
    }
  }

  // B operand: column lc < G is query head kvh*G + lc; k-step s covers dims
  // 32*s + 8*lg .. +8 (the same dims the A lanes load), hi and lo parts.
  h8 qhi[4], qlo[4];
  {
    const bool col = lc < G;
    const float *qsrc = p.q + (size_t)(kvh * G + (col ? lc : 0)) * HD + 8 * lg;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const f4 *src = reinterpret_cast<const f4 *>(qsrc + 32 * s);
      f4 a = src[0], b = src[1];
      float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
      if (FUSED) {
#pragma unroll
        for (int pi = 0; pi < 4; ++pi) {
          float2 cs = sm.cs[16 * s + 4 * lg + pi];
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

  // One 16-key tile starting at key t0; keys >= cend are masked.
  auto process = [&](const TileBuf &b, int t0, int cend) {
    h8 ka[4];
#pragma unroll
    for (int s = 0; s < 4; ++s) ka[s] = __builtin_bit_cast(h8, b.k[s]);
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
  };

  if (n_my > 0) {
    // Ring of kDepth register buffers: tile i+kDepth is requested as soon as
    // tile i has been consumed, so kDepth-1 tiles stay in flight.
    for (int i = 0; i < n_my; i += kDepth) {
#pragma unroll
      for (int b = 0; b < kDepth; ++b) {
        if (i + b < n_my) process(buf[b], (first_tile + kWaves * (i + b)) * kTile, ce);
        issue(buf[b], i + b + kDepth);
      }
    }
  }
  if (has_new && w == 0) {
    // Every row of this tile is the new key / value; only key 0 is unmasked.
    TileBuf nb;
#pragma unroll
    for (int s = 0; s < 4; ++s) nb.k[s] = *reinterpret_cast<const u4 *>(&sm.knew[32 * s + 8 * lg]);
#pragma unroll
    for (int m = 0; m < 4; ++m) nb.v[m] = *reinterpret_cast<const u4 *>(&sm.vnew[8 * lc]);
    process(nb, p.L - 1, p.L);
  }

  // Wave totals: l over the 4 key groups of column lc.
  l_part += __shfl_xor(l_part, 16);
  l_part += __shfl_xor(l_part, 32);
  if (lane < G) {
    sm.ml[w][lane] = m_lane;
    sm.ml[w][G + lane] = l_part;
  }
  if (lc < G) {
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int i = 0; i < 4; ++i) sm.acc[w][lc][8 * (4 * lg + i) + e] = o[e][i];
  }
  __syncthreads();

  constexpr int kOuts = G * HD / kThreads;  // outputs per thread
  float o_val[kOuts], m_wg[kOuts], l_wg[kOuts];
#pragma unroll
  for (int oi = 0; oi < kOuts; ++oi) {
    const int o = tid + oi * kThreads;
    const int g = o / HD, d = o % HD;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) M = fmaxf(M, sm.ml[ww][g]);
    const float Mu = M == -INFINITY ? 0.f : M;
    float Ls = 0.f, O = 0.f;
#pragma unroll
    for (int ww = 0; ww < kWaves; ++ww) {
      float e = fast_exp2(sm.ml[ww][g] - Mu);
      Ls = __builtin_fmaf(e, sm.ml[ww][G + g], Ls);
      O = __builtin_fmaf(e, sm.acc[ww][g][d], O);
    }
    o_val[oi] = O;
    m_wg[oi] = M;
    l_wg[oi] = Ls;
  }

  if (p.nchunk == 1) {
#pragma unroll
    for (int oi = 0; oi < kOuts; ++oi)
      p.out[(size_t)kvh * G * HD + tid + oi * kThreads] = o_val[oi] / l_wg[oi];
    return;
  }

  const size_t pbase = ((size_t)kvh * p.nchunk + chunk) * G;
#pragma unroll
  for (int oi = 0; oi < kOuts; ++oi) {
    const int o = tid + oi * kThreads;
    p.part_o[pbase * HD + o] = o_val[oi];
    if ((o % HD) == 0)
      *reinterpret_cast<float2 *>(p.part_ml + (pbase + o / HD) * 2) = make_float2(m_wg[oi], l_wg[oi]);
  }
}

// Cross-chunk log-sum-exp merge.  Workgroup = (kv head, q head, 32-dim block);
// its 256 threads = 8 chunk groups x 32 dims, so each thread sums about
// nchunk/8 independent partials.  A separate launch: the kernel boundary
// orders the partial writes before these reads, where an in-kernel
// last-arriver merge would need an agent-scope fence (an L2 write-back) in
// every workgroup.
__global__ void __launch_bounds__(256) decode_merge_kernel(DecodeParams p) {
  __shared__ float wt[kMaxChunks];
  __shared__ float red[8][32];
  __shared__ float stat[2];
  const int db = blockIdx.x % 4;
  const int hg = blockIdx.x / 4;  // kvh * G + g
  const int kvh = hg / G, g = hg % G;
  const int tid = threadIdx.x;
  const size_t hb = (size_t)kvh * p.nchunk * G;
  if (tid < 64) {
    float M = -INFINITY;
    for (int c = tid; c < p.nchunk; c += 64) M = fmaxf(M, p.part_ml[(hb + (size_t)c * G + g) * 2]);
    M = wave_max(M);
    float Ls = 0.f;
    for (int c = tid; c < p.nchunk; c += 64) {
      float2 ml = *reinterpret_cast<const float2 *>(p.part_ml + (hb + (size_t)c * G + g) * 2);
      float e = fast_exp2(ml.x - M);
      wt[c] = e;
      Ls = __builtin_fmaf(e, ml.y, Ls);
    }
    Ls = wave_sum(Ls);
    if (tid == 0) stat[0] = 1.0f / Ls;
  }
  __syncthreads();
  const int cg = tid >> 5, d = 32 * db + (tid & 31);
  const float *src = p.part_o + (hb + g) * HD + d;
  float O = 0.f;
#pragma unroll 4
  for (int c = cg; c < p.nchunk; c += 8) O = __builtin_fmaf(wt[c], src[(size_t)c * G * HD], O);
  red[cg][tid & 31] = O;
  __syncthreads();
  if (tid < 32) {
    float t = 0.f;
#pragma unroll
    for (int k = 0; k < 8; ++k) t += red[k][tid];
    p.out[(size_t)hg * HD + d] = t * stat[0];
  }
}

}  // namespace

size_t decode_scratch_bytes(int n_kv, int g, int nchunk) {
  return (size_t)n_kv * nchunk * g * (HD + 2) * sizeof(float);
}

int decode_pick_nchunk(int L, int n_kv, int target_wgs) {
  const int n_tiles = (L + kTile - 1) / kTile;
  // at least one tile per wave, at most kMaxChunks chunks
  int nchunk = (target_wgs + n_kv - 1) / n_kv;
  if (nchunk > n_tiles / kWaves) nchunk = n_tiles / kWaves;
  if (nchunk > kMaxChunks) nchunk = kMaxChunks;
  if (nchunk < 1) nchunk = 1;
  return nchunk;
}

hipError_t launch_decode(const DecodeParams &p, int g, bool fused, hipStream_t s, hipEvent_t ev0,
                         hipEvent_t ev1) {
  if (g != G) return hipErrorInvalidValue;
  if (p.nchunk < 1 || p.nchunk > kMaxChunks) return hipErrorInvalidValue;
  dim3 grid(p.n_kv * p.nchunk), block(kThreads);
  if (fused)
    hipExtLaunchKernelGGL(decode_kernel<true>, grid, block, 0, s, ev0, ev1, 0, p);
  else
    hipExtLaunchKernelGGL(decode_kernel<false>, grid, block, 0, s, ev0, ev1, 0, p);
  return hipGetLastError();
}

hipError_t launch_decode_merge(const DecodeParams &p, hipStream_t s) {
  if (p.nchunk > 1) hipLaunchKernelGGL(decode_merge_kernel, dim3(p.n_kv * G * 4), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace mia
