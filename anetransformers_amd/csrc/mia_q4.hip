// mia_q4.hip -- the W4A8 projections either side of the attention step:
// fp32 -> Q8_0 quantisation of an activation vector (mistral/dequant.h:545-612)
// and the Q4_0 x Q8_0 matvec (mistral/dequant.h:1022-1137), for one matrix or
// for the Q, K and V matrices in one launch (mistral_model.h:676-745).
//
// Block formats (mistral/dequant.h:17-31, 535-541):
//   Q4_0  18 B per 32 weights: fp16 scale, then 16 bytes; byte j holds weight j
//         in its low nibble and weight j+16 in its high nibble, each stored +8.
//   Q8_0  36 B per 32 values: fp32 scale, then 32 int8.
//
// Matvec layout: a row is bpr * 18 bytes with bpr even, so every pair of
// blocks is 36 bytes at a 4-byte aligned offset.  Lane l of a wave takes block
// pairs l, l+64, ... of each of the R rows the wave owns, loads all R rows and
// the matching 72 bytes of x before using any of them, and forms each block's
// integer dot with v_dot4 on the raw nibbles (0..15 are valid int8) minus
// 8 * sum(x block): the same integer as sum((nibble - 8) * x).  Each block term
// is (wd * xd) * (float)isum, rounded as in the reference; the terms of a row
// are then summed per lane and across the wave (the reference sums them in
// block order, so rows agree to fp32 reassociation, not bit for bit).
#include "mia_device.h"
#include "mia_kernels.h"

namespace mia {
namespace {

constexpr int kQ4Threads = 512;
constexpr int kQ4Waves = kQ4Threads / 64;
static_assert(kQ4Waves == 8, "the RMSNorm prologue combines eight wave sums");
constexpr unsigned kNib = 0x0F0F0F0Fu;

__device__ __forceinline__ unsigned ld32(const uint8_t *p) {
  return *reinterpret_cast<const unsigned *>(p);
}

__device__ __forceinline__ float f16_bits(unsigned h) {
  return (float)__builtin_bit_cast(_Float16, (unsigned short)(h & 0xFFFFu));
}

__device__ __forceinline__ int dot4(unsigned a, unsigned b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float *__restrict__ x,
                                                            uint8_t *__restrict__ out,
                                                            int nblocks) {
  const int gid = blockIdx.x * 256 + threadIdx.x;
  const int blk = gid >> 3, sub = gid & 7;
  if (blk >= nblocks) return;  // whole 8-lane groups leave together
  const f4 v = *reinterpret_cast<const f4 *>(x + (size_t)blk * 32 + sub * 4);
  q8_block_part(v, sub, out + (size_t)blk * 36);
}

// XP > 0: x is fp32 and every workgroup quantises it into LDS (the same
// arithmetic as quantize_q8_0_kernel, so the blocks are bit-identical) while
// its weight rows are in flight; each thread loads XP groups of 4 values, so
// XP * kQ4Threads / 8 >= bpr.  XP = 0: x is Q8_0 blocks in global memory.
// PRO (XP > 0 only): 1 RMS-normalises x before quantising it, 2 forms the
// SwiGLU product gate * sigmoid(gate) * up from x = gate (Q4MatvecParams).
// Thread t holds x's 4-value groups at 4t + 2048k, so its sum of squares, the
// wave sums and their fixed combination are rmsnorm_kernel's own, and the
// normalised values equal launch_rmsnorm's bit for bit.
template <int R, int XP, int PRO>
__global__ __launch_bounds__(kQ4Threads) void q4_matvec_kernel(Q4MatvecParams p) {
#pragma clang fp contract(off)
  constexpr bool kF32X = XP > 0;
  __shared__ __attribute__((aligned(16))) uint8_t xq_lds[kF32X ? XP * (kQ4Threads / 8) * 36 : 4];
  __shared__ float red[kQ4Waves];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = (blockIdx.x * kQ4Waves + wave) * R;
  const size_t row_bytes = (size_t)p.bpr * 18;

  // Virtual rows 0..rows0-1 are w0's, then w1's, then w2's.  Rows past the
  // end load the last row (in bounds) and store nothing.
  const uint8_t *wrow[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int g = min(row0 + r, p.total_rows - 1);
    const uint8_t *base = g < p.rows0 ? p.w0 : (g < p.rows01 ? p.w1 : p.w2);
    const int lr = g < p.rows0 ? g : (g < p.rows01 ? g - p.rows0 : g - p.rows01);
    wrow[r] = p.swiglu ? ((g & 1) ? p.w1 : p.w0) + (size_t)(g >> 1) * row_bytes
                       : base + (size_t)lr * row_bytes;
  }

  const int npairs = p.bpr >> 1;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.0f;
  unsigned wv[R][9];
  auto load_rows = [&](int pc) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const uint8_t *wp = wrow[r] + (size_t)pc * 36;
#pragma unroll
      for (int j = 0; j < 9; ++j) wv[r][j] = ld32(wp + 4 * j);
    }
  };

  if constexpr (kF32X) {
    // Activation loads first (clamped in bounds), then the first weight
    // rows: waiting for the activations then leaves the rows in flight.
    f4 xr[XP], ar[PRO ? XP : 1];
#pragma unroll
    for (int k = 0; k < XP; ++k) {
      const int blk = min(k * (kQ4Threads / 8) + (int)(threadIdx.x >> 3), p.bpr - 1);
      const size_t off = (size_t)blk * 32 + (threadIdx.x & 7) * 4;
      xr[k] = *reinterpret_cast<const f4 *>(p.xf + off);
      if constexpr (PRO == 1) ar[k] = *reinterpret_cast<const f4 *>(p.rms_w + off);
      if constexpr (PRO == 2) ar[k] = *reinterpret_cast<const f4 *>(p.up + off);
    }
    __builtin_amdgcn_sched_barrier(0);
    load_rows(min(lane, npairs - 1));
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (PRO == 1) {
      // rmsnorm_vec (mistral_model.h:202-208) of the whole x
      float ss = 0.0f;
#pragma unroll
      for (int k = 0; k < XP; ++k) {
        const f4 v = xr[k];
        if (k * (kQ4Threads / 8) + (int)(threadIdx.x >> 3) < p.bpr)
          ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
      }
      ss = wave_sum(ss);
      if (lane == 0) red[wave] = ss;
      __syncthreads();
      ss = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
      const float scale = 1.0f / sqrtf(ss / (float)(p.bpr * 32) + p.eps);
#pragma unroll
      for (int k = 0; k < XP; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) xr[k][e] = (xr[k][e] * scale) * ar[k][e];
    }
    if constexpr (PRO == 2) {
      // silu_mul_neon (mistral_model.h:174-199)
#pragma unroll
      for (int k = 0; k < XP; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float g = xr[k][e];
          const float sig = 1.0f / (1.0f + expf(-g));
          xr[k][e] = (g * sig) * ar[k][e];
        }
    }
#pragma unroll
    for (int k = 0; k < XP; ++k) {
      const int blk = k * (kQ4Threads / 8) + (int)(threadIdx.x >> 3);
      if (blk < p.bpr)  // whole 8-lane groups
        q8_block_part(xr[k], threadIdx.x & 7, xq_lds + blk * 36);
    }
    // LDS writes done and visible; the weight loads stay outstanding.
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  }

  for (int p0 = 0; p0 < npairs; p0 += 64) {
    const int pr = p0 + lane;
    const bool on = pr < npairs;
    const int pc = on ? pr : npairs - 1;
    if (!kF32X || p0 > 0) load_rows(pc);
    unsigned xv[18];
    if constexpr (kF32X) {
      const uint8_t *xp = xq_lds + pc * 72;
#pragma unroll
      for (int j = 0; j < 18; ++j) xv[j] = *reinterpret_cast<const unsigned *>(xp + 4 * j);
    } else {
      const uint8_t *xp = p.x + (size_t)pc * 72;
#pragma unroll
      for (int j = 0; j < 18; ++j) xv[j] = ld32(xp + 4 * j);
    }

    // x block A: d = xv[0], qs = xv[1..8]; block B: d = xv[9], qs = xv[10..17]
    int sxa = 0, sxb = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      sxa = dot4(xv[1 + i], 0x01010101u, sxa);
      sxb = dot4(xv[10 + i], 0x01010101u, sxb);
    }
    const float xda = __builtin_bit_cast(float, xv[0]);
    const float xdb = __builtin_bit_cast(float, xv[9]);

#pragma unroll
    for (int r = 0; r < R; ++r) {
      const unsigned *w = wv[r];
      // weight block A: scale in bytes 0-1, nibbles in bytes 2-17
      int ia = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const unsigned q = __builtin_amdgcn_alignbyte(w[i + 1], w[i], 2);
        ia = dot4(q & kNib, xv[1 + i], ia);
        ia = dot4((q >> 4) & kNib, xv[5 + i], ia);
      }
      ia -= 8 * sxa;
      // weight block B: scale in bytes 18-19, nibbles in bytes 20-35
      int ib = 0;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const unsigned q = w[5 + i];
        ib = dot4(q & kNib, xv[10 + i], ib);
        ib = dot4((q >> 4) & kNib, xv[14 + i], ib);
      }
      ib -= 8 * sxb;
      const float ta = (f16_bits(w[0]) * xda) * (float)ia;
      const float tb = (f16_bits(w[4] >> 16) * xdb) * (float)ib;
      acc[r] += on ? ta + tb : 0.0f;
    }
  }

  float sum[R];
#pragma unroll
  for (int r = 0; r < R; ++r) sum[r] = wave_sum(acc[r]);
  if (p.swiglu) {
    static_assert(R == 2, "a wave holds one gate row and its up row");
    // silu_mul_neon (mistral_model.h:174-199) of row j's gate and up sums
    if (lane == 0 && row0 < p.total_rows) {
      const float g = sum[0];
      const float sig = 1.0f / (1.0f + expf(-g));
      p.y0[row0 >> 1] = (g * sig) * sum[1];
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int g = row0 + r;
    if (lane == 0 && g < p.total_rows) {
      float *y = g < p.rows0 ? p.y0 + g : (g < p.rows01 ? p.y1 + (g - p.rows0) : p.y2 + (g - p.rows01));
      *y = p.resid ? p.resid[g] + sum[r] : sum[r];
    }
  }
}

}  // namespace

hipError_t launch_quantize_q8_0(const float *x, uint8_t *out, int nblocks, hipStream_t s) {
  const int threads = nblocks * 8;
  hipLaunchKernelGGL(quantize_q8_0_kernel, dim3((threads + 255) / 256), dim3(256), 0, s, x, out,
                     nblocks);
  return hipGetLastError();
}

template <int PRO>
hipError_t launch_q4_xp(const Q4MatvecParams &p, dim3 grid, hipStream_t s, hipEvent_t ev0,
                        hipEvent_t ev1) {
  constexpr int R = 2;
  constexpr int kBlocksPerPass = kQ4Threads / 8;
  static_assert(8 * kBlocksPerPass * 32 >= kQ4MaxFusedInDim, "fused passes cover the inputs");
  if (p.bpr * 32 > kQ4MaxFusedInDim) return hipErrorInvalidValue;
  if (p.bpr <= kBlocksPerPass)
    hipExtLaunchKernelGGL((q4_matvec_kernel<R, 1, PRO>), grid, dim3(kQ4Threads), 0, s, ev0, ev1,
                          0, p);
  else if (p.bpr <= 2 * kBlocksPerPass)
    hipExtLaunchKernelGGL((q4_matvec_kernel<R, 2, PRO>), grid, dim3(kQ4Threads), 0, s, ev0, ev1,
                          0, p);
  else if (p.bpr <= 4 * kBlocksPerPass)
    hipExtLaunchKernelGGL((q4_matvec_kernel<R, 4, PRO>), grid, dim3(kQ4Threads), 0, s, ev0, ev1,
                          0, p);
  else
    hipExtLaunchKernelGGL((q4_matvec_kernel<R, 8, PRO>), grid, dim3(kQ4Threads), 0, s, ev0, ev1,
                          0, p);
  return hipGetLastError();
}

hipError_t launch_q4_matvec(const Q4MatvecParams &p, hipStream_t s, hipEvent_t ev0,
                            hipEvent_t ev1) {
  constexpr int R = 2;
  const int rows_per_wg = kQ4Waves * R;
  const dim3 grid((p.total_rows + rows_per_wg - 1) / rows_per_wg);
  if (!p.xf) {
    if (p.rms_w || p.up) return hipErrorInvalidValue;
    hipExtLaunchKernelGGL((q4_matvec_kernel<R, 0, 0>), grid, dim3(kQ4Threads), 0, s, ev0, ev1, 0,
                          p);
    return hipGetLastError();
  }
  if (p.rms_w && p.up) return hipErrorInvalidValue;
  if (p.rms_w) return launch_q4_xp<1>(p, grid, s, ev0, ev1);
  if (p.up) return launch_q4_xp<2>(p, grid, s, ev0, ev1);
  return launch_q4_xp<0>(p, grid, s, ev0, ev1);
}

}  // namespace mia
