// mia_prefill.hip -- the rest of the prefill layer around the attention step
// (mistral/mistral_ane_prefill.h:1081-1110): RMSNorm of the token rows
// (:163-175) and the Q4_0 GEMM on fp32 activations (:999-1042, the reference
// dequantises 128-row tiles to fp32 and calls cblas_sgemm), with epilogues for
// the residual adds and SwiGLU (mistral_model.h:174-199).
//
// GEMM: Y[S][N] = X[S][K] . W[N][K]^T on fp16 MFMA (v_mfma_f32_32x32x16_f16)
// with fp32 accuracy where it matters:
//   - X is split into fp16 hi + lo (x = hi + lo to ~2^-22) as it is staged
//     into LDS, and both halves go through the MFMA;
//   - W's 4-bit values q - 8 are exact in fp16; the fp16 block scale d is
//     applied in fp32 once per 32-value block: acc += d * (X . q) for the
//     block's partial product, which is what dequantising to fp32 computes.
// Workgroup: 256 threads, 128 tokens x 64 weight rows, 4 waves of 64 x 32;
// each iteration stages 64 K values (two Q4_0 blocks, 36 bytes of each row,
// 4-byte aligned because the blocks per row are even) through one LDS buffer,
// with the next iteration's global loads in registers during the MFMAs.
#include "mia_device.h"
#include "mia_kernels.h"

namespace mia {
namespace {

constexpr int kGThreads = 256;
constexpr int kBM = 128;          // tokens per workgroup
constexpr int kBN = 64;           // weight rows per workgroup
constexpr int kBK = 64;           // K values per iteration (two Q4_0 blocks)
constexpr int kKP = kBK + 8;      // LDS row stride in halves (144 B: conflict-free b128 reads)

struct GemmLds {
  _Float16 ahi[kBM][kKP];
  _Float16 alo[kBM][kKP];
  _Float16 bq[kBN][kKP];
  float bd[kBN][2];
};

__device__ __forceinline__ float f16_bits_f32(unsigned h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
}

// Two 4-bit values n0, n1 (in bits 0-3 and 16-19 of v) -> fp16 (n0 - 8, n1 - 8):
// 0x6400 | n is the fp16 number 1024 + n, and 1024 + n - 1032 is exact.
__device__ __forceinline__ unsigned nib2_to_h2(unsigned v) {
  typedef _Float16 h2 __attribute__((ext_vector_type(2)));
  const h2 x = __builtin_bit_cast(h2, v | 0x64006400u);
  const h2 r = x - (h2){(_Float16)1032.0f, (_Float16)1032.0f};
  return __builtin_bit_cast(unsigned, r);
}

template <int MODE>
__global__ __launch_bounds__(kGThreads) void q4_gemm_kernel(GemmParams p) {
#pragma clang fp contract(off)
  __shared__ __attribute__((aligned(16))) GemmLds sm;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave >> 1, wn = wave & 1;
  const int n0 = blockIdx.x * kBN, m0 = blockIdx.y * kBM;

  // A staging: thread -> token row ar, 32 values at column ac of the iteration
  const int ar = tid >> 1, ac = 32 * (tid & 1);
  const float *aptr = p.A + (size_t)min(m0 + ar, p.S - 1) * p.lda + ac;
  // B staging: thread -> weight row br, block bb (0, 1) of the iteration's pair
  const int br = tid & (kBN - 1), bb = (tid >> 6) & 1;
  const bool bload = tid < 2 * kBN;
  const uint8_t *bptr;
  {
    const int g = min(n0 + br, p.N - 1);
    const uint8_t *base = g < p.rows0 ? p.w0 : (g < p.rows01 ? p.w1 : p.w2);
    const int lr = g < p.rows0 ? g : (g < p.rows01 ? g - p.rows0 : g - p.rows01);
    bptr = base + (size_t)lr * (size_t)(p.K / 32) * 18 + 16 * bb;
  }

  f4 areg[8];
  unsigned breg[5];
  auto load = [&](int it) {
    const float *a = aptr + (size_t)it * kBK;
#pragma unroll
    for (int j = 0; j < 8; ++j) areg[j] = *reinterpret_cast<const f4 *>(a + 4 * j);
    if (bload) {
      const uint8_t *b = bptr + (size_t)it * 36;
#pragma unroll
      for (int j = 0; j < 5; ++j) breg[j] = *reinterpret_cast<const unsigned *>(b + 4 * j);
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      h8 hi, lo;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float x = e < 4 ? areg[j][e] : areg[j + 1][e - 4];
        const _Float16 h = (_Float16)x;
        hi[e] = h;
        lo[e] = (_Float16)(x - (float)h);
      }
      *reinterpret_cast<h8 *>(&sm.ahi[ar][ac + 4 * j]) = hi;
      *reinterpret_cast<h8 *>(&sm.alo[ar][ac + 4 * j]) = lo;
    }
    if (bload) {
      // bb 0: bytes 0-19 of the pair (scale 0-1, nibbles 2-17);
      // bb 1: bytes 16-35 (scale 18-19, nibbles 20-35)
      unsigned q[4];
      float d;
      if (bb == 0) {
        d = f16_bits_f32(breg[0]);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = __builtin_amdgcn_alignbyte(breg[i + 1], breg[i], 2);
      } else {
        d = f16_bits_f32(breg[0] >> 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) q[i] = breg[i + 1];
      }
      // byte j: low nibble = value j, high nibble = value j + 16
      unsigned lo8[8], hi8[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const unsigned v = q[i], h = q[i] >> 4;
        lo8[2 * i] = nib2_to_h2((v & 0xFu) | ((v << 8) & 0xF0000u));
        lo8[2 * i + 1] = nib2_to_h2(((v >> 16) & 0xFu) | ((v >> 8) & 0xF0000u));
        hi8[2 * i] = nib2_to_h2((h & 0xFu) | ((h << 8) & 0xF0000u));
        hi8[2 * i + 1] = nib2_to_h2(((h >> 16) & 0xFu) | ((h >> 8) & 0xF0000u));
      }
      _Float16 *dst = &sm.bq[br][32 * bb];
      *reinterpret_cast<u4 *>(dst) = (u4){lo8[0], lo8[1], lo8[2], lo8[3]};
      *reinterpret_cast<u4 *>(dst + 8) = (u4){lo8[4], lo8[5], lo8[6], lo8[7]};
      *reinterpret_cast<u4 *>(dst + 16) = (u4){hi8[0], hi8[1], hi8[2], hi8[3]};
      *reinterpret_cast<u4 *>(dst + 24) = (u4){hi8[4], hi8[5], hi8[6], hi8[7]};
      sm.bd[br][bb] = d;
    }
  };

  f16v acc[2];
#pragma unroll
  for (int t = 0; t < 2; ++t)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[t][i] = 0.0f;

  const int n_it = p.K / kBK;
  const int col = lane & 31, half = lane >> 5;
  load(0);
  for (int it = 0; it < n_it; ++it) {
    __syncthreads();  // the previous iteration's operand reads are done
    store();
    __syncthreads();
    if (it + 1 < n_it) load(it + 1);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      f16v blk[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int k = 32 * kb + 16 * ks + 8 * half;
        const h8 b = *reinterpret_cast<const h8 *>(&sm.bq[32 * wn + col][k]);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          const int r = 64 * wm + 32 * t + col;
          const h8 ah = *reinterpret_cast<const h8 *>(&sm.ahi[r][k]);
          const h8 al = *reinterpret_cast<const h8 *>(&sm.alo[r][k]);
          if (ks == 0) {
#pragma unroll
            for (int i = 0; i < 16; ++i) blk[t][i] = 0.0f;
          }
          blk[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, b, blk[t], 0, 0, 0);
          blk[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, b, blk[t], 0, 0, 0);
        }
      }
      const float d = sm.bd[32 * wn + col][kb];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < 16; ++i) acc[t][i] = __builtin_fmaf(d, blk[t][i], acc[t][i]);
    }
  }

  // D layout: lane holds column n = col; value i is row 8*(i/4) + 4*half + i%4.
  const int n = n0 + 32 * wn + col;
  if (n >= p.N) return;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const int m = m0 + 64 * wm + 32 * t + 8 * (i >> 2) + 4 * half + (i & 3);
      if (m >= p.S) continue;
      const float v = acc[t][i];
      if (MODE == kGemmStore) {
        if (n < p.rows0)
          p.y0[(size_t)m * p.rows0 + n] = v;
        else if (n < p.rows01)
          p.y1[(size_t)m * (p.rows01 - p.rows0) + (n - p.rows0)] = v;
        else
          p.y2[(size_t)m * (p.N - p.rows01) + (n - p.rows01)] = v;
      } else if (MODE == kGemmAdd) {
        float *y = p.y0 + (size_t)m * p.N + n;
        *y = *y + v;
      } else {  // kGemmSiluMul: y0 holds the gate; gate * sigmoid(gate) * up
        float *y = p.y0 + (size_t)m * p.N + n;
        const float g = *y;
        const float sig = 1.0f / (1.0f + expf(-g));
        *y = (g * sig) * v;
      }
    }
  }
}

// One workgroup per token row: ss = sum(x^2), scale = 1 / sqrt(ss / dim + eps),
// out = (x * scale) * w, the reference's two roundings (vsmul then vmul).
__global__ __launch_bounds__(256) void rmsnorm_kernel(float *out, const float *in, const float *w,
                                                      int dim, float eps) {
  __shared__ float red[4];
  const int t = blockIdx.x, tid = threadIdx.x;
  const float *x = in + (size_t)t * dim;
  float ss = 0.0f;
  for (int i = 4 * tid; i < dim; i += 4 * 256) {
    const f4 v = *reinterpret_cast<const f4 *>(x + i);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  ss = (red[0] + red[1]) + (red[2] + red[3]);
  const float scale = 1.0f / sqrtf(ss / (float)dim + eps);
  float *o = out + (size_t)t * dim;
  for (int i = 4 * tid; i < dim; i += 4 * 256) {
    const f4 v = *reinterpret_cast<const f4 *>(x + i);
    const f4 wv = *reinterpret_cast<const f4 *>(w + i);
    f4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = (v[e] * scale) * wv[e];
    *reinterpret_cast<f4 *>(o + i) = r;
  }
}

}  // namespace

hipError_t launch_q4_gemm(const GemmParams &p, int mode, hipStream_t s, hipEvent_t ev0,
                          hipEvent_t ev1) {
  const dim3 grid((p.N + kBN - 1) / kBN, (p.S + kBM - 1) / kBM);
  if (mode == kGemmStore)
    hipExtLaunchKernelGGL(q4_gemm_kernel<kGemmStore>, grid, dim3(kGThreads), 0, s, ev0, ev1, 0, p);
  else if (mode == kGemmAdd)
    hipExtLaunchKernelGGL(q4_gemm_kernel<kGemmAdd>, grid, dim3(kGThreads), 0, s, ev0, ev1, 0, p);
  else
    hipExtLaunchKernelGGL(q4_gemm_kernel<kGemmSiluMul>, grid, dim3(kGThreads), 0, s, ev0, ev1, 0,
                          p);
  return hipGetLastError();
}

hipError_t launch_rmsnorm(float *out, const float *in, const float *w, int dim, int S, float eps,
                          hipStream_t s) {
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(S), dim3(256), 0, s, out, in, w, dim, eps);
  return hipGetLastError();
}

}  // namespace mia
