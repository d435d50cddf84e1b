// mia_decode.hip -- S=1 GQA decode attention for gfx950 (split-K flash-decode).
//
// Replaces mistral/mistral_model.h:362-487 (gqa_attention_neon), and, in the
// fused variant, steps 4-6 of mistral/mistral_model.h:849-863 (RoPE on q/k,
// fp16 round of k/v, ring write at pos % max_seq, attention).
//
// Grid: one workgroup per (kv head, chunk of the window); blockIdx % n_kv is
// the kv head so that, with the hardware's round-robin workgroup dispatch over
// the 8 XCDs, every chunk of one kv head (and its partials) stays on one XCD.
//
// Workgroup = 4 waves; each wave owns 64-row slices of the chunk.  Inside a
// wave a 16-lane DPP row handles one cache row: lane j holds dims 8j..8j+7, so
// a wave load instruction fetches 4 rows x 256 contiguous bytes, and each
// loaded fp16 element is used by all G query heads of the group from
// registers (v_fma_mix_f32, no conversion instructions).  Scores of a 64-row
// slice go through LDS once (one lane per row) for the wave-level online
// softmax; the 4 wave partials are merged in LDS, and chunk partials are merged
// by the last-arriving workgroup of the kv head (log-sum-exp merge).
#include "mia_device.h"
#include "mia_kernels.h"

namespace mia {

namespace {

constexpr int kThreads = 256;
constexpr int kBlockRows = 256;  // rows per workgroup pass (4 waves x 64)
constexpr int kGroups = 16;      // 4-row load groups per wave slice
constexpr int kMaxChunks = 256;  // merge capacity per kv head

template <int G>
struct DecodeSmem {
  float2 cs[64];               // RoPE (cos, sin) for the 64 pair indices
  float p[4][64][G];           // per-wave slice scores -> probabilities
  float ml[4][2 * G];          // per-wave (max, sum)
  int last;
  union {
    float acc[4][4][G][HD];    // per-(wave, row group) partial outputs
    struct {
      float2 mlc[kMaxChunks * G];
      float wt[kMaxChunks * G];
      float2 fin[G];
    } merge;
  } u;
};

template <int G>
__device__ __forceinline__ void load_row_vec(const float *src, float (&v)[G]) {
#pragma unroll
  for (int g = 0; g < G; ++g) v[g] = src[g];
}

template <int G, bool FUSED>
__global__ void __launch_bounds__(kThreads, 2) decode_kernel(DecodeParams p) {
  static_assert(G == 4, "decode kernel is instantiated for 4 query heads per kv head");
  __shared__ DecodeSmem<G> sm;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int w = tid >> 6;
  const int r = lane >> 4;  // row within a 4-row load group
  const int j = lane & 15;  // dims 8j..8j+7
  const int kvh = blockIdx.x % p.n_kv;
  const int chunk = blockIdx.x / p.n_kv;
  const int kv_dim = p.n_kv * HD;
  const int c0 = chunk * p.chunk_rows;
  const int c1 = min(c0 + p.chunk_rows, p.L);
  const bool has_new = FUSED && (c1 == p.L);

  if (FUSED) {
    if (tid < 64) {
      // angle = fl32(theta_inv[i] * pos) as vDSP_vsmul (mistral_model.h:87-88)
      float ang = p.theta_inv[tid] * (float)p.pos;
      float sn, cs;
      sincosf(ang, &sn, &cs);
      sm.cs[tid] = make_float2(cs, sn);
    }
    __syncthreads();
  }

  // q of the G heads sharing this kv head, dims 8j..8j+7, rotated and scaled.
  float q[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const f4 *src = reinterpret_cast<const f4 *>(p.q + (size_t)(kvh * G + g) * HD + 8 * j);
    f4 a = src[0], b = src[1];
    float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
    if (FUSED) {
#pragma unroll
      for (int pi = 0; pi < 4; ++pi) {
        float2 cs = sm.cs[4 * j + pi];
        rope_pair(v[2 * pi], v[2 * pi + 1], cs.x, cs.y);
      }
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) q[g][e] = v[e] * p.qscale;
  }

  // The new token's fp16 k/v for this kv head (only the last chunk uses it).
  h8 kn16 = {}, vn16 = {};
  if (has_new) {
    const f4 *ks = reinterpret_cast<const f4 *>(p.knew + (size_t)kvh * HD + 8 * j);
    const f4 *vs = reinterpret_cast<const f4 *>(p.vnew + (size_t)kvh * HD + 8 * j);
    f4 a = ks[0], b = ks[1];
    float kv8[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
    for (int pi = 0; pi < 4; ++pi) {
      float2 cs = sm.cs[4 * j + pi];
      rope_pair(kv8[2 * pi], kv8[2 * pi + 1], cs.x, cs.y);
    }
    f4 va = vs[0], vb = vs[1];
    float vv8[8] = {va.x, va.y, va.z, va.w, vb.x, vb.y, vb.z, vb.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      kn16[e] = (_Float16)kv8[e];  // RNE, as vcvt_f16_f32 (mistral_model.h:854)
      vn16[e] = (_Float16)vv8[e];
    }
    if (tid < 16) {  // one 256-B row per tensor: kv_write at pos % max_seq
      size_t off = (size_t)p.new_slot * kv_dim + (size_t)kvh * HD + 8 * j;
      *reinterpret_cast<u4 *>(p.kc + off) = __builtin_bit_cast(u4, kn16);
      *reinterpret_cast<u4 *>(p.vc + off) = __builtin_bit_cast(u4, vn16);
    }
  }

  float m_run[G], l_run[G], acc[G][8];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_run[g] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[g][e] = 0.f;
  }

  const _Float16 *kbase = p.kc + (size_t)kvh * HD + 8 * j;
  const _Float16 *vbase = p.vc + (size_t)kvh * HD + 8 * j;

  for (int b0 = c0; b0 < c1; b0 += kBlockRows) {
    const int rb = b0 + w * 64;  // first row of this wave's slice
    if (rb >= c1) break;         // wave-uniform: nothing left for this wave

    u4 kd[kGroups], vd[kGroups];
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      int t = min(rb + g * 4 + r, c1 - 1);
      int slot = p.start + t;
      slot = slot >= p.max_seq ? slot - p.max_seq : slot;
      unsigned off = (unsigned)slot * (unsigned)kv_dim;
      kd[g] = *reinterpret_cast<const u4 *>(kbase + off);
    }
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      int t = min(rb + g * 4 + r, c1 - 1);
      int slot = p.start + t;
      slot = slot >= p.max_seq ? slot - p.max_seq : slot;
      unsigned off = (unsigned)slot * (unsigned)kv_dim;
      vd[g] = *reinterpret_cast<const u4 *>(vbase + off);
    }

    // Scores: 8-dim partial dots per lane, summed over the 16-lane row.
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      const int t = rb + g * 4 + r;
      h8 kh = __builtin_bit_cast(h8, kd[g]);
      if (has_new && t == p.L - 1) kh = kn16;
      float d[G];
#pragma unroll
      for (int gg = 0; gg < G; ++gg) d[gg] = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float kf = (float)kh[e];
#pragma unroll
        for (int gg = 0; gg < G; ++gg) d[gg] = __builtin_fmaf(q[gg][e], kf, d[gg]);
      }
#pragma unroll
      for (int gg = 0; gg < G; ++gg) d[gg] = row16_sum(d[gg]);
      if (j == 0) {
        const bool valid = t < c1;
        f4 sv = {valid ? d[0] : -INFINITY, valid ? d[1] : -INFINITY,
                 valid ? d[2] : -INFINITY, valid ? d[3] : -INFINITY};
        *reinterpret_cast<f4 *>(&sm.p[w][g * 4 + r][0]) = sv;
      }
    }
    wave_lds_sync();

    // Wave-level online softmax over the slice (one row per lane).
    {
      f4 sc = *reinterpret_cast<const f4 *>(&sm.p[w][lane][0]);
      float s[G] = {sc.x, sc.y, sc.z, sc.w};
      float pr[G];
#pragma unroll
      for (int gg = 0; gg < G; ++gg) {
        float mb = wave_max(s[gg]);
        float mn = fmaxf(m_run[gg], mb);
        float alpha = fast_exp2(m_run[gg] - mn);
        pr[gg] = fast_exp2(s[gg] - mn);
        float lb = wave_sum(pr[gg]);
        l_run[gg] = l_run[gg] * alpha + lb;
        m_run[gg] = mn;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[gg][e] *= alpha;
      }
      f4 pv = {pr[0], pr[1], pr[2], pr[3]};
      *reinterpret_cast<f4 *>(&sm.p[w][lane][0]) = pv;
    }
    wave_lds_sync();

    // Weighted V sum.
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      const int t = rb + g * 4 + r;
      f4 pp = *reinterpret_cast<const f4 *>(&sm.p[w][g * 4 + r][0]);
      float pw[G] = {pp.x, pp.y, pp.z, pp.w};
      h8 vh = __builtin_bit_cast(h8, vd[g]);
      if (has_new && t == p.L - 1) vh = vn16;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float vf = (float)vh[e];
#pragma unroll
        for (int gg = 0; gg < G; ++gg) acc[gg][e] = __builtin_fmaf(pw[gg], vf, acc[gg][e]);
      }
    }
    wave_lds_sync();
  }

  // Merge the 4 waves x 4 row groups inside the workgroup.
  if (lane == 0) {
#pragma unroll
    for (int gg = 0; gg < G; ++gg) {
      sm.ml[w][gg] = m_run[gg];
      sm.ml[w][G + gg] = l_run[gg];
    }
  }
#pragma unroll
  for (int gg = 0; gg < G; ++gg) {
    f4 *dst = reinterpret_cast<f4 *>(&sm.u.acc[w][r][gg][8 * j]);
    dst[0] = f4{acc[gg][0], acc[gg][1], acc[gg][2], acc[gg][3]};
    dst[1] = f4{acc[gg][4], acc[gg][5], acc[gg][6], acc[gg][7]};
  }
  __syncthreads();

  constexpr int kOuts = G * HD / kThreads;  // outputs per thread
  float o_val[kOuts], m_wg[kOuts], l_wg[kOuts];
#pragma unroll
  for (int oi = 0; oi < kOuts; ++oi) {
    const int o = tid + oi * kThreads;
    const int gg = o / HD, d = o % HD;
    float M = -INFINITY;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) M = fmaxf(M, sm.ml[ww][gg]);
    float Ls = 0.f, O = 0.f;
#pragma unroll
    for (int ww = 0; ww < 4; ++ww) {
      float e = fast_exp2(sm.ml[ww][gg] - M);
      Ls = __builtin_fmaf(e, sm.ml[ww][G + gg], Ls);
      float s = (sm.u.acc[ww][0][gg][d] + sm.u.acc[ww][1][gg][d]) +
                (sm.u.acc[ww][2][gg][d] + sm.u.acc[ww][3][gg][d]);
      O = __builtin_fmaf(e, s, O);
    }
    o_val[oi] = O;
    m_wg[oi] = M;
    l_wg[oi] = Ls;
  }

  if (p.nchunk == 1) {
#pragma unroll
    for (int oi = 0; oi < kOuts; ++oi) {
      const int o = tid + oi * kThreads;
      p.out[(size_t)kvh * G * HD + o] = o_val[oi] / l_wg[oi];
    }
    return;
  }

  const size_t pbase = ((size_t)kvh * p.nchunk + chunk) * G;
#pragma unroll
  for (int oi = 0; oi < kOuts; ++oi) {
    const int o = tid + oi * kThreads;
    p.part_o[pbase * HD + o] = o_val[oi];
    if ((o % HD) == 0) {
      const int gg = o / HD;
      *reinterpret_cast<float2 *>(p.part_ml + (pbase + gg) * 2) = make_float2(m_wg[oi], l_wg[oi]);
    }
  }

  // Last-arriving workgroup of this kv head merges all chunk partials.
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    unsigned prev = atomicAdd(&p.counter[kvh], 1u);
    sm.last = (prev == (unsigned)(p.nchunk - 1));
  }
  __syncthreads();
  if (!sm.last) return;
  __threadfence();

  const size_t hbase = (size_t)kvh * p.nchunk * G;
  for (int i = tid; i < p.nchunk * G; i += kThreads)
    sm.u.merge.mlc[i] = *reinterpret_cast<const float2 *>(p.part_ml + (hbase + i) * 2);
  __syncthreads();
  if (tid < G) {
    float M = -INFINITY;
    for (int c = 0; c < p.nchunk; ++c) M = fmaxf(M, sm.u.merge.mlc[c * G + tid].x);
    float Ls = 0.f;
    for (int c = 0; c < p.nchunk; ++c) {
      float2 ml = sm.u.merge.mlc[c * G + tid];
      Ls = __builtin_fmaf(fast_exp2(ml.x - M), ml.y, Ls);
    }
    sm.u.merge.fin[tid] = make_float2(M, 1.0f / Ls);
  }
  __syncthreads();
  for (int i = tid; i < p.nchunk * G; i += kThreads) {
    float2 fin = sm.u.merge.fin[i % G];
    sm.u.merge.wt[i] = fast_exp2(sm.u.merge.mlc[i].x - fin.x) * fin.y;
  }
  __syncthreads();
#pragma unroll
  for (int oi = 0; oi < kOuts; ++oi) {
    const int o = tid + oi * kThreads;
    const int gg = o / HD;
    float O = 0.f;
    const float *src = p.part_o + hbase * HD + o;
    int c = 0;
    for (; c + 4 <= p.nchunk; c += 4) {
      float a0 = src[(size_t)(c + 0) * G * HD], a1 = src[(size_t)(c + 1) * G * HD];
      float a2 = src[(size_t)(c + 2) * G * HD], a3 = src[(size_t)(c + 3) * G * HD];
      O = __builtin_fmaf(sm.u.merge.wt[(c + 0) * G + gg], a0, O);
      O = __builtin_fmaf(sm.u.merge.wt[(c + 1) * G + gg], a1, O);
      O = __builtin_fmaf(sm.u.merge.wt[(c + 2) * G + gg], a2, O);
      O = __builtin_fmaf(sm.u.merge.wt[(c + 3) * G + gg], a3, O);
    }
    for (; c < p.nchunk; ++c) O = __builtin_fmaf(sm.u.merge.wt[c * G + gg], src[(size_t)c * G * HD], O);
    p.out[(size_t)kvh * G * HD + o] = O;
  }
  if (tid == 0) atomicExch(&p.counter[kvh], 0u);
}

}  // namespace

size_t decode_scratch_bytes(int n_kv, int G, int nchunk) {
  return (size_t)n_kv * nchunk * G * (HD + 2) * sizeof(float);
}

int decode_pick_chunk_rows(int L, int n_kv, int target_wgs) {
  long per = ((long)L * n_kv + target_wgs - 1) / target_wgs;
  long rows = ((per + kBlockRows - 1) / kBlockRows) * kBlockRows;
  if (rows < kBlockRows) rows = kBlockRows;
  long nchunk = (L + rows - 1) / rows;
  while (nchunk > kMaxChunks) {
    rows += kBlockRows;
    nchunk = (L + rows - 1) / rows;
  }
  return (int)rows;
}

hipError_t launch_decode(const DecodeParams &p, int G, bool fused, hipStream_t s) {
  if (G != 4) return hipErrorInvalidValue;
  if (p.nchunk > kMaxChunks || p.chunk_rows % kBlockRows) return hipErrorInvalidValue;
  dim3 grid(p.n_kv * p.nchunk), block(kThreads);
  if (fused)
    hipLaunchKernelGGL((decode_kernel<4, true>), grid, block, 0, s, p);
  else
    hipLaunchKernelGGL((decode_kernel<4, false>), grid, block, 0, s, p);
  return hipGetLastError();
}

}  // namespace mia
