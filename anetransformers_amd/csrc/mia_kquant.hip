// mia_kquant.hip -- the weight types other than Q4_0 that the reference's
// projections and prefill GEMM accept: Q4_K and Q6_K (its Q4_K_M target),
// F16 and F32 (mistral/mistral_model.h:211-243, 581-670;
// mistral/mistral_ane_prefill.h:907-1042).
//
// The reference multiplies these weights in fp32 after dequantising them:
//   Q4_K  per 32-value sub-block, in fp16 arithmetic (dequant_q4_K_block_neon,
//         dequant.h:68-125): vd = fp16(d * sc), vm = fp16(dmin * m),
//         w = fp16(fp16(q * vd) - vm)
//   Q6_K  w = (d * scales[n / 16]) * (q - 32) in fp32 (dequant_q6_K_block,
//         dequant.h:291-307), value n taken from ql / qh as that function does
//   Q4_0  (prefill GEMM only) w = d * (q - 8) in fp32 (mistral_ane_prefill.h:921-939)
// Every kernel here forms those weights bit for bit, 32 consecutive values
// of a row at a time (a "group": a Q4_K sub-block, two Q6_K sub-blocks, a
// Q4_0 block), and then
//   typed_matvec_kernel   y = W . x, one wave per row, lane l taking the row's
//                         groups l, l + 64, ...; x fp32 or Q8_0 blocks (the
//                         reference's non-Q4_0 decode path dequantises its
//                         Q8_0 activations, mistral_model.h:656-670); fp32
//                         fma per lane, then a wave sum (the reference's
//                         sgemv / four-lane NEON sums in another order)
//   typed_dequant_kernel  the fp32 weight rows, for the prefill GEMM, which
//                         the library then hands to the BLAS library's sgemm
//                         as the reference does (mistral_ane_prefill.h:1018-1042)
// Memory-bound like the Q4_0 matvec: 0.5625 (Q4_K), 0.82 (Q6_K), 2 or 4
// bytes per weight.
#include "mia_device.h"
#include "mia_kernels.h"

namespace mia {

namespace {

constexpr int kQKK = 256;    // values per Q4_K / Q6_K super-block
constexpr int kQ4KBytes = 144;
constexpr int kQ6KBytes = 210;

__device__ __forceinline__ float half_bits(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}

__device__ __forceinline__ uint16_t load_u16(const uint8_t *p) {
  return (uint16_t)(p[0] | (p[1] << 8));
}

// Group g (32 values) of a row in the type's layout -> v[32], the weights the
// reference multiplies.
template <int TYPE>
__device__ __forceinline__ void dequant_group(const uint8_t *row, int g, float (&v)[32]) {
#pragma clang fp contract(off)
  if constexpr (TYPE == kTypeQ4K) {
    const uint8_t *blk = row + (size_t)(g >> 3) * kQ4KBytes;
    const int j = g & 7;  // sub-block
    const float d = half_bits(load_u16(blk)), dmin = half_bits(load_u16(blk + 2));
    const uint8_t *sc = blk + 4;
    // get_scale_min_k4 (dequant.h:58-66)
    int s, m;
    if (j < 4) {
      s = sc[j] & 63;
      m = sc[j + 4] & 63;
    } else {
      s = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4);
      m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
    }
    const _Float16 vd = (_Float16)(d * (float)s), vm = (_Float16)(dmin * (float)m);
    // low nibbles of qs[32 (j / 2) ..] for even j, high nibbles for odd j
    const uint8_t *qs = blk + 16 + 32 * (j >> 1);
    const int sh = (j & 1) * 4;
    u4 raw[2];
    raw[0] = *reinterpret_cast<const u4 *>(qs);
    raw[1] = *reinterpret_cast<const u4 *>(qs + 16);
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      const unsigned byte = (raw[l >> 4][(l >> 2) & 3] >> (8 * (l & 3))) & 0xFF;
      const _Float16 p = (_Float16)(float)((byte >> sh) & 0xF) * vd;
      const _Float16 o = p - vm;
      v[l] = (float)o;
    }
  } else if constexpr (TYPE == kTypeQ6K) {
    const uint8_t *blk = row + (size_t)(g >> 3) * kQ6KBytes;
    const int n0 = 32 * (g & 7);
    const uint8_t *ql = blk + (n0 < 128 ? n0 : n0 - 128);
    const uint8_t *qh = blk + 128 + (n0 & 63);
    const int lo_sh = n0 < 128 ? 0 : 4;
    // qh bit pair: 0 (n < 64), 4 (64..127), 2 (128..191), 6 (192..255)
    const int r = n0 >> 6;
    const int hi_sh = r == 0 ? 0 : (r == 1 ? 4 : (r == 2 ? 2 : 6));
    const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192);
    const float d = half_bits(load_u16(blk + 208));
    const float ds0 = d * (float)sc[n0 >> 4], ds1 = d * (float)sc[(n0 >> 4) + 1];
#pragma unroll
    for (int l = 0; l < 32; ++l) {
      const int q = (((ql[l] >> lo_sh) & 0xF) | (((qh[l] >> hi_sh) & 3) << 4)) - 32;
      v[l] = (l < 16 ? ds0 : ds1) * (float)q;
    }
  } else if constexpr (TYPE == kTypeQ40) {
    const uint8_t *blk = row + (size_t)g * 18;
    const float d = half_bits(load_u16(blk));
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const unsigned b = blk[2 + i];
      v[i] = d * ((float)(b & 0x0F) - 8.0f);
      v[i + 16] = d * ((float)(b >> 4) - 8.0f);
    }
  } else if constexpr (TYPE == kTypeF16) {
    const u4 *src = reinterpret_cast<const u4 *>(row + (size_t)g * 64);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const h8 h = __builtin_bit_cast(h8, src[k]);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[8 * k + e] = (float)h[e];
    }
  } else {  // F32
    const f4 *src = reinterpret_cast<const f4 *>(row + (size_t)g * 128);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const f4 x = src[k];
      v[4 * k] = x.x;
      v[4 * k + 1] = x.y;
      v[4 * k + 2] = x.z;
      v[4 * k + 3] = x.w;
    }
  }
}

template <int TYPE, bool XQ8>
__global__ void __launch_bounds__(512) typed_matvec_kernel(const uint8_t *W, long row_bytes,
                                                           const void *x, float *y, int rows,
                                                           int cols) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 8 + (threadIdx.x >> 6);
  if (row >= rows) return;  // whole wave
  const uint8_t *wr = W + (size_t)row * row_bytes;
  const int ngroups = cols >> 5;
  float acc = 0.f;
  for (int g = lane; g < ngroups; g += 64) {
    float w[32];
    dequant_group<TYPE>(wr, g, w);
    if constexpr (XQ8) {
      // Q8_0 block g: fp32 d, 32 int8 (36 bytes); the reference's x value is
      // d * q in fp32 (mistral_model.h:662-666)
      // (blocks are 4-byte aligned only: dword loads)
      const unsigned *blk = reinterpret_cast<const unsigned *>(
          reinterpret_cast<const uint8_t *>(x) + (size_t)g * 36);
      const float d = __builtin_bit_cast(float, blk[0]);
      unsigned qw[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) qw[k] = blk[1 + k];
#pragma unroll
      for (int l = 0; l < 32; ++l) {
        const int q = (int)(signed char)((qw[l >> 2] >> (8 * (l & 3))) & 0xFF);
        acc = __builtin_fmaf(w[l], d * (float)q, acc);
      }
    } else {
      const f4 *xs = reinterpret_cast<const f4 *>(reinterpret_cast<const float *>(x) + 32 * g);
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const f4 xv = xs[k];
        acc = __builtin_fmaf(w[4 * k], xv.x, acc);
        acc = __builtin_fmaf(w[4 * k + 1], xv.y, acc);
        acc = __builtin_fmaf(w[4 * k + 2], xv.z, acc);
        acc = __builtin_fmaf(w[4 * k + 3], xv.w, acc);
      }
    }
  }
  acc = wave_sum(acc);
  if (lane == 0) y[row] = acc;
}

// One thread per group: 32 fp32 weights of a row.
template <int TYPE>
__global__ void __launch_bounds__(256) typed_dequant_kernel(const uint8_t *W, long row_bytes,
                                                            float *out, int rows, int cols) {
  const int ngroups = cols >> 5;
  const long total = (long)rows * ngroups;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    const int r = (int)(i / ngroups), g = (int)(i % ngroups);
    float w[32];
    dequant_group<TYPE>(W + (size_t)r * row_bytes, g, w);
    f4 *dst = reinterpret_cast<f4 *>(out + (size_t)r * cols + 32 * g);
#pragma unroll
    for (int k = 0; k < 8; ++k) dst[k] = (f4){w[4 * k], w[4 * k + 1], w[4 * k + 2], w[4 * k + 3]};
  }
}

// mistral_model.h:174-199 (silu_mul_neon): gate = gate * (1 / (1 + exp(-gate))) * up
__global__ void __launch_bounds__(256) silu_mul_kernel(float *gate, const float *up, long n) {
#pragma clang fp contract(off)
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < n; i += (long)gridDim.x * 256) {
    const float g = gate[i];
    const float sig = 1.0f / (1.0f + expf(-g));
    gate[i] = (g * sig) * up[i];
  }
}

template <int TYPE>
hipError_t launch_matvec_t(const void *W, long rb, const void *x, bool xq8, float *y, int rows,
                           int cols, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  const dim3 grid((rows + 7) / 8), block(512);
  const uint8_t *w = reinterpret_cast<const uint8_t *>(W);
  if (xq8)
    hipExtLaunchKernelGGL((typed_matvec_kernel<TYPE, true>), grid, block, 0, s, ev0, ev1, 0, w,
                          rb, x, y, rows, cols);
  else
    hipExtLaunchKernelGGL((typed_matvec_kernel<TYPE, false>), grid, block, 0, s, ev0, ev1, 0, w,
                          rb, x, y, rows, cols);
  return hipGetLastError();
}

template <int TYPE>
hipError_t launch_dequant_t(const void *W, long rb, float *out, int rows, int cols,
                            hipStream_t s) {
  const long total = (long)rows * (cols >> 5);
  long blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL((typed_dequant_kernel<TYPE>), dim3((unsigned)blocks), dim3(256), 0, s,
                     reinterpret_cast<const uint8_t *>(W), rb, out, rows, cols);
  return hipGetLastError();
}

}  // namespace

long typed_row_bytes(int type, int cols) {
  if (cols <= 0 || cols % 32) return 0;
  switch (type) {
    case kTypeF32: return (long)cols * 4;
    case kTypeF16: return (long)cols * 2;
    case kTypeQ40: return (long)(cols / 32) * 18;
    case kTypeQ4K: return cols % kQKK ? 0 : (long)(cols / kQKK) * kQ4KBytes;
    case kTypeQ6K: return cols % kQKK ? 0 : (long)(cols / kQKK) * kQ6KBytes;
    default: return 0;
  }
}

hipError_t launch_typed_matvec(const void *W, int type, const void *x, bool x_q8, float *y,
                               int rows, int cols, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  const long rb = typed_row_bytes(type, cols);
  if (rb == 0 || rows <= 0) return hipErrorInvalidValue;
  switch (type) {
    case kTypeQ4K: return launch_matvec_t<kTypeQ4K>(W, rb, x, x_q8, y, rows, cols, s, ev0, ev1);
    case kTypeQ6K: return launch_matvec_t<kTypeQ6K>(W, rb, x, x_q8, y, rows, cols, s, ev0, ev1);
    case kTypeF16: return launch_matvec_t<kTypeF16>(W, rb, x, x_q8, y, rows, cols, s, ev0, ev1);
    case kTypeF32: return launch_matvec_t<kTypeF32>(W, rb, x, x_q8, y, rows, cols, s, ev0, ev1);
    case kTypeQ40: return launch_matvec_t<kTypeQ40>(W, rb, x, x_q8, y, rows, cols, s, ev0, ev1);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_typed_dequant(const void *W, int type, float *out, int rows, int cols,
                                hipStream_t s) {
  const long rb = typed_row_bytes(type, cols);
  if (rb == 0 || rows <= 0) return hipErrorInvalidValue;
  switch (type) {
    case kTypeQ40: return launch_dequant_t<kTypeQ40>(W, rb, out, rows, cols, s);
    case kTypeQ4K: return launch_dequant_t<kTypeQ4K>(W, rb, out, rows, cols, s);
    case kTypeQ6K: return launch_dequant_t<kTypeQ6K>(W, rb, out, rows, cols, s);
    case kTypeF16: return launch_dequant_t<kTypeF16>(W, rb, out, rows, cols, s);
    case kTypeF32: return launch_dequant_t<kTypeF32>(W, rb, out, rows, cols, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_silu_mul(float *gate, const float *up, long n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  long blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, s, gate, up, n);
  return hipGetLastError();
}

}  // namespace mia
