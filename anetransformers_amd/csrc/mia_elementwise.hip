// mia_elementwise.hip -- RoPE, fp32->fp16 ring writes, staging commit and the
// synthetic-input fills used by the benchmark.
#include "mia_device.h"
#include "mia_kernels.h"

namespace mia {

namespace {

// One thread per (token, pair index); rotates that pair in every q and k head.
// mistral/mistral_model.h:79-122 and mistral/mistral_ane_prefill.h:177-186.
__global__ void rope_kernel(float *q, float *k, int S, int start_pos, const float *theta_inv,
                            int n_heads, int n_kv) {
  const int t = blockIdx.x;
  const int i = threadIdx.x;  // pair index < 64
  if (t >= S || i >= HD / 2) return;
  float ang = theta_inv[i] * (float)(start_pos + t);
  float sn, cs;
  sincosf(ang, &sn, &cs);
  if (q) {
    float *qt = q + (size_t)t * n_heads * HD;
    for (int h = 0; h < n_heads; ++h) {
      float2 v = *reinterpret_cast<float2 *>(qt + h * HD + 2 * i);
      rope_pair(v.x, v.y, cs, sn);
      *reinterpret_cast<float2 *>(qt + h * HD + 2 * i) = v;
    }
  }
  if (k) {
    float *kt = k + (size_t)t * n_kv * HD;
    for (int h = 0; h < n_kv; ++h) {
      float2 v = *reinterpret_cast<float2 *>(kt + h * HD + 2 * i);
      rope_pair(v.x, v.y, cs, sn);
      *reinterpret_cast<float2 *>(kt + h * HD + 2 * i) = v;
    }
  }
}

// One workgroup of 128 threads per token.  The 64 (cos, sin) pairs of the
// token's position, fl32(theta_inv[i] * pos) as vDSP_vsmul + vvsincosf
// (mistral_model.h:87-90), are formed once and optionally stored to cs_out for
// the attention kernel's Q rotation.  Each thread then rotates 8 consecutive
// dims (4 adjacent pairs, mistral_model.h:100-105) of one kv head of K, rounds
// K and V to fp16 (RNE, mistral_model.h:160-169) and writes them to the ring
// slot pos % max_seq (kv_write, kv_cache.h:53-57) or to a dense staging row.
// With more tokens than ring slots, token t shares its slot with t + max_seq:
// the reference writes in token order (kv_write_batch), so tokens
// t < S - max_seq write nothing (their (cos, sin) rows are still stored).
__global__ void __launch_bounds__(128)
    rope_kv_f16_kernel(const float *K, const float *V, const float *theta_inv, int S, int start_pos,
                       int n_kv, _Float16 *kdst, _Float16 *vdst, int max_seq, bool ring,
                       float *cs_out) {
  __shared__ float2 cs[HD / 2];
  const int t = blockIdx.x;
  const int tid = threadIdx.x;
  const int pos = start_pos + t;
  const int kv_dim = n_kv * HD;
  const int n_items = n_kv * (HD / 8);
  // The K/V loads of the thread's first item are issued before the angles
  // are formed, so that their latency overlaps the sincos and the barrier.
  f4 k0 = {}, k1 = {}, v0 = {}, v1 = {};
  if (tid < n_items) {
    const int e0 = (tid >> 4) * HD + 8 * (tid & 15);
    const f4 *ks = reinterpret_cast<const f4 *>(K + (size_t)t * kv_dim + e0);
    const f4 *vs = reinterpret_cast<const f4 *>(V + (size_t)t * kv_dim + e0);
    k0 = ks[0];
    k1 = ks[1];
    v0 = vs[0];
    v1 = vs[1];
  }
  if (tid < HD / 2) {
    const float ang = theta_inv[tid] * (float)pos;
    float sn, c;
    sincosf(ang, &sn, &c);
    cs[tid] = make_float2(c, sn);
    if (cs_out) reinterpret_cast<float2 *>(cs_out)[(size_t)t * (HD / 2) + tid] = make_float2(c, sn);
  }
  __syncthreads();
  if (ring && t < S - max_seq) return;
  const size_t drow = ring ? (size_t)(pos % max_seq) : (size_t)t;
  for (int c = tid; c < n_items; c += blockDim.x) {
    const int e0 = (c >> 4) * HD + 8 * (c & 15);
    if (c != tid) {
      const f4 *ks = reinterpret_cast<const f4 *>(K + (size_t)t * kv_dim + e0);
      const f4 *vs = reinterpret_cast<const f4 *>(V + (size_t)t * kv_dim + e0);
      k0 = ks[0];
      k1 = ks[1];
      v0 = vs[0];
      v1 = vs[1];
    }
    float kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    const int p0 = 4 * (c & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float2 q = cs[p0 + i];
      rope_pair(kk[2 * i], kk[2 * i + 1], q.x, q.y);
    }
    h8 kh, vh;
#pragma unroll
    for (int i = 0; i < 8; ++i) kh[i] = (_Float16)kk[i];
    vh[0] = (_Float16)v0.x; vh[1] = (_Float16)v0.y; vh[2] = (_Float16)v0.z; vh[3] = (_Float16)v0.w;
    vh[4] = (_Float16)v1.x; vh[5] = (_Float16)v1.y; vh[6] = (_Float16)v1.z; vh[7] = (_Float16)v1.w;
    *reinterpret_cast<h8 *>(kdst + drow * kv_dim + e0) = kh;
    *reinterpret_cast<h8 *>(vdst + drow * kv_dim + e0) = vh;
  }
}

// Long chunks: the last token of each slot, found in one linear pass.
// owner[slot] holds -1 between calls; every token claims its slot with an
// atomic max of its index, and rope_kv_positions_kernel resets the slot
// after reading it.
__global__ void slot_claim_kernel(const int *positions, int S, int max_seq, int *owner) {
  const int t = blockIdx.x * blockDim.x + threadIdx.x;
  if (t >= S) return;
  const int pos = positions[t];
  if (pos >= 0) atomicMax(owner + pos % max_seq, t);
}

// Phase 1 of the chunked prefill for K / V (mistral/mistral_model.h:935-955):
// one workgroup of 128 threads per token t.  k is rotated at positions[t]
// (angles fl32(theta_inv[i] * pos), mistral_model.h:87-105), k and v are
// rounded to fp16 and written to slot positions[t] % max_seq -- unless a
// later token of the chunk takes the same slot: the reference writes the
// tokens in order, so that later token is what the slot keeps.  Without
// `owner` each token looks for such a later token among positions[t+1..S)
// (short chunks); with it, the slot_claim_kernel launch before this one has
// left the slot's last token there: the token that finds itself writes and
// puts -1 back (a token that reads -1 there is not the last either).
__global__ void __launch_bounds__(128)
    rope_kv_positions_kernel(const float *K, const float *V, const float *theta_inv,
                             const int *positions, int S, int n_kv, _Float16 *kc, _Float16 *vc,
                             int max_seq, int *owner) {
  __shared__ float2 cs[HD / 2];
  __shared__ int overwritten;
  const int t = blockIdx.x;
  const int tid = threadIdx.x;
  const int pos = positions[t];
  if (pos < 0) return;  // no slot (the attention gives such a token a zero row)
  const int slot = pos % max_seq;
  if (owner != nullptr) {
    if (tid == 0) {
      const int last = owner[slot];
      overwritten = last != t;
      if (last == t) owner[slot] = -1;
    }
  } else {
    if (tid == 0) overwritten = 0;
    __syncthreads();
    for (int u = t + 1 + tid; u < S; u += blockDim.x) {
      const int pu = positions[u];
      if (pu >= 0 && pu % max_seq == slot) overwritten = 1;
    }
  }
  if (tid < HD / 2) {
    const float ang = theta_inv[tid] * (float)pos;
    float sn, c;
    sincosf(ang, &sn, &c);
    cs[tid] = make_float2(c, sn);
  }
  __syncthreads();
  if (overwritten) return;  // workgroup-uniform
  const int kv_dim = n_kv * HD;
  for (int c = tid; c < n_kv * (HD / 8); c += blockDim.x) {
    const int e0 = (c >> 4) * HD + 8 * (c & 15);
    const f4 *ks = reinterpret_cast<const f4 *>(K + (size_t)t * kv_dim + e0);
    const f4 *vs = reinterpret_cast<const f4 *>(V + (size_t)t * kv_dim + e0);
    const f4 k0 = ks[0], k1 = ks[1], v0 = vs[0], v1 = vs[1];
    float kk[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    const int p0 = 4 * (c & 15);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float2 q = cs[p0 + i];
      rope_pair(kk[2 * i], kk[2 * i + 1], q.x, q.y);
    }
    h8 kh, vh;
#pragma unroll
    for (int i = 0; i < 8; ++i) kh[i] = (_Float16)kk[i];
    vh[0] = (_Float16)v0.x; vh[1] = (_Float16)v0.y; vh[2] = (_Float16)v0.z; vh[3] = (_Float16)v0.w;
    vh[4] = (_Float16)v1.x; vh[5] = (_Float16)v1.y; vh[6] = (_Float16)v1.z; vh[7] = (_Float16)v1.w;
    *reinterpret_cast<h8 *>(kc + (size_t)slot * kv_dim + e0) = kh;
    *reinterpret_cast<h8 *>(vc + (size_t)slot * kv_dim + e0) = vh;
  }
}

// mistral/mistral_ane_prefill.h:189-204: cvt + kv_write at (start+t) % M.
// The reference writes the tokens in order, so with S > M a slot keeps the
// last token written to it: tokens t < S - M are overwritten and skipped here
// (several blocks writing one slot at once would leave any of them).
__global__ void kv_write_kernel(_Float16 *kc, _Float16 *vc, const float *K, const float *V, int S,
                                int start_pos, int max_seq, int kv_dim) {
  const int t = blockIdx.y;
  if (t < S - max_seq) return;
  const size_t slot = (size_t)((start_pos + t) % max_seq);
  for (int e = blockIdx.x * blockDim.x + threadIdx.x; e < kv_dim; e += gridDim.x * blockDim.x) {
    kc[slot * kv_dim + e] = (_Float16)K[(size_t)t * kv_dim + e];
    vc[slot * kv_dim + e] = (_Float16)V[(size_t)t * kv_dim + e];
  }
}

// Staged row t of layer blockIdx.z -> ring slot (start_pos + t) % max_seq of
// that layer; layers are ring_stride / stage_stride elements apart.  Rows a
// later row overwrites (t < S - max_seq) are skipped: the sequential writes
// leave the last one.
__global__ void commit_kernel(_Float16 *kc, _Float16 *vc, const _Float16 *kst,
                              const _Float16 *vst, int S, int start_pos, int max_seq, int kv_dim,
                              size_t ring_stride, size_t stage_stride) {
  const int t = blockIdx.y;
  if (t < S - max_seq) return;
  const size_t slot = (size_t)((start_pos + t) % max_seq);
  kc += blockIdx.z * ring_stride;
  vc += blockIdx.z * ring_stride;
  kst += blockIdx.z * stage_stride;
  vst += blockIdx.z * stage_stride;
  for (int e = (blockIdx.x * blockDim.x + threadIdx.x) * 8; e < kv_dim;
       e += gridDim.x * blockDim.x * 8) {
    *reinterpret_cast<u4 *>(kc + slot * kv_dim + e) =
        *reinterpret_cast<const u4 *>(kst + (size_t)t * kv_dim + e);
    *reinterpret_cast<u4 *>(vc + slot * kv_dim + e) =
        *reinterpret_cast<const u4 *>(vst + (size_t)t * kv_dim + e);
  }
}

__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
  x += 0x9E3779B97F4A7C15ull;
  x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
  x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
  return x ^ (x >> 31);
}

// N(0,1) via Box-Muller on a counter-based splitmix64 stream, rounded to fp16.
__global__ void fill_normal_kernel(_Float16 *dst, size_t n, uint64_t seed) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x) {
    uint64_t r = splitmix64(seed ^ (i * 0xD1B54A32D192ED03ull));
    float u1 = ((float)(r >> 40) + 1.0f) * (1.0f / 16777216.0f);  // (0, 1]
    float u2 = (float)((r >> 16) & 0xFFFFFFu) * (1.0f / 16777216.0f);
    float z = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
    dst[i] = (_Float16)z;
  }
}

__global__ void scale_rows_kernel(_Float16 *base, long n_rows, int row_elems, int every, int offset,
                                  float factor) {
  const long n_sel = (n_rows - offset + every - 1) / every;
  const long total = n_sel * row_elems;
  for (long i = (long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (long)gridDim.x * blockDim.x) {
    long rr = offset + (i / row_elems) * every;
    long e = i % row_elems;
    _Float16 *pp = base + rr * row_elems + e;
    *pp = (_Float16)((float)*pp * factor);
  }
}

}  // namespace

hipError_t launch_rope(float *q, float *k, int S, int start_pos, const float *theta_inv,
                       int n_heads, int n_kv, hipStream_t s) {
  if (S <= 0) return hipSuccess;
  hipLaunchKernelGGL(rope_kernel, dim3(S), dim3(64), 0, s, q, k, S, start_pos, theta_inv, n_heads,
                     n_kv);
  return hipGetLastError();
}

hipError_t launch_rope_to_f16(const float *K, const float *V, const float *theta_inv, int S,
                              int start_pos, int n_kv, _Float16 *kdst, _Float16 *vdst,
                              float *cs_out, hipStream_t s) {
  if (S <= 0) return hipSuccess;
  hipLaunchKernelGGL(rope_kv_f16_kernel, dim3(S), dim3(128), 0, s, K, V, theta_inv, S, start_pos,
                     n_kv, kdst, vdst, 1, false, cs_out);
  return hipGetLastError();
}

hipError_t launch_rope_to_ring(const float *K, const float *V, const float *theta_inv, int S,
                               int start_pos, int n_kv, _Float16 *kc, _Float16 *vc, int max_seq,
                               float *cs_out, hipStream_t s) {
  if (S <= 0) return hipSuccess;
  hipLaunchKernelGGL(rope_kv_f16_kernel, dim3(S), dim3(128), 0, s, K, V, theta_inv, S, start_pos,
                     n_kv, kc, vc, max_seq, true, cs_out);
  return hipGetLastError();
}

hipError_t launch_kv_write(_Float16 *kc, _Float16 *vc, const float *K, const float *V, int S,
                           int start_pos, int max_seq, int kv_dim, hipStream_t s) {
  if (S <= 0) return hipSuccess;
  int bx = (kv_dim + 255) / 256;
  hipLaunchKernelGGL(kv_write_kernel, dim3(bx, S), dim3(256), 0, s, kc, vc, K, V, S, start_pos,
                     max_seq, kv_dim);
  return hipGetLastError();
}

hipError_t launch_rope_kv_positions(const float *K, const float *V, const float *theta_inv,
                                    const int *positions, int S, int n_kv, _Float16 *kc,
                                    _Float16 *vc, int max_seq, int *owner, hipStream_t s) {
  if (S <= 0) return hipSuccess;
  if (owner != nullptr) {
    hipLaunchKernelGGL(slot_claim_kernel, dim3((S + 255) / 256), dim3(256), 0, s, positions, S,
                       max_seq, owner);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  hipLaunchKernelGGL(rope_kv_positions_kernel, dim3(S), dim3(128), 0, s, K, V, theta_inv,
                     positions, S, n_kv, kc, vc, max_seq, owner);
  return hipGetLastError();
}

hipError_t launch_commit(_Float16 *kc, _Float16 *vc, const _Float16 *kst, const _Float16 *vst,
                         int S, int start_pos, int max_seq, int kv_dim, hipStream_t s,
                         int n_layers, size_t ring_stride, size_t stage_stride) {
  if (S <= 0 || n_layers <= 0) return hipSuccess;
  int bx = (kv_dim / 8 + 127) / 128;
  hipLaunchKernelGGL(commit_kernel, dim3(bx, S, n_layers), dim3(128), 0, s, kc, vc, kst, vst, S,
                     start_pos, max_seq, kv_dim, ring_stride, stage_stride);
  return hipGetLastError();
}

hipError_t launch_fill_normal(_Float16 *dst, size_t n, uint64_t seed, hipStream_t s) {
  if (n == 0) return hipSuccess;
  size_t blocks = (n + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  hipLaunchKernelGGL(fill_normal_kernel, dim3((unsigned)blocks), dim3(256), 0, s, dst, n, seed);
  return hipGetLastError();
}

hipError_t launch_scale_rows(_Float16 *base, long n_rows, int row_elems, int every, int offset,
                             float factor, hipStream_t s) {
  if (n_rows <= offset || every <= 0) return hipSuccess;
  hipLaunchKernelGGL(scale_rows_kernel, dim3(4096), dim3(256), 0, s, base, n_rows, row_elems,
                     every, offset, factor);
  return hipGetLastError();
}

}  // namespace mia
