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
//   Q4_0  w = d * (q - 8) in fp32 (q4_0_matvec_f32, dequant.h:142-278;
//         mistral_ane_prefill.h:921-939)
// Every kernel here forms those weights bit for bit, 32 consecutive values of
// a row at a time (a "group": a Q4_K sub-block, two Q6_K sub-blocks, a Q4_0
// block):
//   kquant_matvec_kernel  y = W . x for Q4_K / Q6_K, x fp32 or Q8_0 blocks
//                         (the reference's non-Q4_0 decode path dequantises
//                         its Q8_0 activations, mistral_model.h:656-670); R
//                         rows per wave sharing the lane's x values
//   typed_matvec_kernel   the same for F16, F32 and Q4_0 with fp32 x, one
//                         wave per row
//   typed_dequant_kernel  the fp32 weight rows (dequant_weight_to_fp32_buf)
//   typed_split_kernel    the prefill GEMM's fp16 operands: the fp16 values of
//                         Q4_K / F16 weights, row-scaled hi + lo halves of
//                         Q6_K / F32 weights, for rocBLAS gemm_ex
//   hilo_combine_kernel   the GEMM's partial products summed (+ residual)
//   silu_mul_kernel       the SwiGLU product between the FFN GEMMs
// Every matvec row sums its fp32 products in another order than the
// reference's sgemv / four-lane NEON sums.  The matvecs are memory-bound:
// 0.5625 (Q4_K), 0.82 (Q6_K), 2 or 4 bytes per weight.
#include <type_traits>

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

typedef _Float16 h2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ u4 load_u4_unaligned(const uint8_t *p) {
  u4 v;
  __builtin_memcpy(&v, p, 16);
  return v;
}

// The K-quant matvec: each wave takes R consecutive rows and lane l the
// 32-value groups l, l + 64, ... of all of them (with Q8_0 inputs the group
// pairs l, l + 64, ..., kq_load_pair), so that the lane's x values are loaded
// (and, from Q8_0 blocks, formed) once for R rows.
//   Q4_K: the group's 32 nibbles as packed fp16 pairs (0x6400 | n is
//         1024 + n), then p = fl16(n * vd) as one packed fma, (1024 + n) * vd
//         - 1024 * vd, whose exact value is n * vd (1024 * vd is exact in
//         fp16 while |vd| <= 63.5; otherwise 1024 is subtracted first), and
//         w = fl16(p - vm): every weight is the reference's; fp32 fma against x.
//   Q6_K: the values q - 32 as fp32 (exact), sum_k q_k x_k per 16-value
//         sub-block, times d * scale: w = d * scale * q is exact in fp32
//         (11 + 7 + 5 significant bits), so this is the reference's sum
//         reassociated.

template <int E>
__device__ __forceinline__ float ubyte_f32(unsigned q) {
  float f;
  if constexpr (E == 0) asm("v_cvt_f32_ubyte0 %0, %1" : "=v"(f) : "v"(q));
  if constexpr (E == 1) asm("v_cvt_f32_ubyte1 %0, %1" : "=v"(f) : "v"(q));
  if constexpr (E == 2) asm("v_cvt_f32_ubyte2 %0, %1" : "=v"(f) : "v"(q));
  if constexpr (E == 3) asm("v_cvt_f32_ubyte3 %0, %1" : "=v"(f) : "v"(q));
  return f;
}

// A group's raw bytes, loaded for every row before any is used.
struct Q4KRaw {
  u4 hdr, qa, qb;
};
struct Q6KRaw {
  u4 ql0, ql1, qh0, qh1;
  unsigned sc2;  // the two int8 scales of the group's sub-blocks
  unsigned dh;   // fp16 d
};

__device__ __forceinline__ void kq_load(const uint8_t *row, int g, Q4KRaw &r) {
  const uint8_t *blk = row + (size_t)(g >> 3) * kQ4KBytes;
  const int j = g & 7;
  r.hdr = *reinterpret_cast<const u4 *>(blk);
  r.qa = *reinterpret_cast<const u4 *>(blk + 16 + 32 * (j >> 1));
  r.qb = *reinterpret_cast<const u4 *>(blk + 32 + 32 * (j >> 1));
}

__device__ __forceinline__ void kq_load(const uint8_t *row, int g, Q6KRaw &r) {
  const uint8_t *blk = row + (size_t)(g >> 3) * kQ6KBytes;
  const int n0 = 32 * (g & 7);
  const uint8_t *qlp = blk + (n0 < 128 ? n0 : n0 - 128);
  const uint8_t *qhp = blk + 128 + (n0 & 63);
  r.ql0 = load_u4_unaligned(qlp);
  r.ql1 = load_u4_unaligned(qlp + 16);
  r.qh0 = load_u4_unaligned(qhp);
  r.qh1 = load_u4_unaligned(qhp + 16);
  r.sc2 = load_u16(blk + 192 + (n0 >> 4));
  r.dh = load_u16(blk + 208);
}

__device__ __forceinline__ float kq_dot(const Q4KRaw &raw, int g, const float (&x)[32]) {
#pragma clang fp contract(off)
  const int j = g & 7;
  const u4 hdr = raw.hdr;
  const float d = half_bits(hdr[0] & 0xFFFF), dmin = half_bits(hdr[0] >> 16);
  // get_scale_min_k4 (dequant.h:58-66): the bytes sit at position j % 4 of
  // the words holding scale bytes 0-3, 4-7 and 8-11
  const int p8 = 8 * (j & 3);
  const unsigned x1 = hdr[1] >> p8, x2 = hdr[2] >> p8, x3 = hdr[3] >> p8;
  const unsigned sv = j < 4 ? (x1 & 63) : ((x3 & 0xF) | ((x1 >> 2) & 0x30));
  const unsigned mv = j < 4 ? (x2 & 63) : (((x3 >> 4) & 0xF) | ((x2 >> 2) & 0x30));
  const _Float16 vd = (_Float16)(d * (float)sv), vm = (_Float16)(dmin * (float)mv);
  const h2 vd2 = {vd, vd}, vm2 = {vm, vm};
  const _Float16 c = (_Float16)-1024.0f * vd;
  const h2 c2 = {c, c}, k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  const int sh = 4 * (j & 1);
  const unsigned magic = 0x64006400u;
  const bool fast = __all(__builtin_fabsf((float)vd) <= 63.5f);
  const u4 qv[2] = {raw.qa, raw.qb};
  float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const unsigned t = qv[i >> 2][i & 3] >> sh;
    // bytes 0, 2 and bytes 1, 3 of the word: values 4i, 4i + 2 and 4i + 1, 4i + 3
    unsigned ua, ub;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(ua) : "v"(t), "s"(0x000F000Fu), "v"(magic));
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(ub) : "v"(t >> 8), "s"(0x000F000Fu), "v"(magic));
    const h2 na = __builtin_bit_cast(h2, ua), nb = __builtin_bit_cast(h2, ub);
    h2 pa, pb;
    if (fast) {
      pa = __builtin_elementwise_fma(na, vd2, c2);
      pb = __builtin_elementwise_fma(nb, vd2, c2);
    } else {
      pa = (na - k1024) * vd2;
      pb = (nb - k1024) * vd2;
    }
    const h2 wa = pa - vm2, wb = pb - vm2;
    acc0 = __builtin_fmaf((float)wa[0], x[4 * i], acc0);
    acc1 = __builtin_fmaf((float)wb[0], x[4 * i + 1], acc1);
    acc0 = __builtin_fmaf((float)wa[1], x[4 * i + 2], acc0);
    acc1 = __builtin_fmaf((float)wb[1], x[4 * i + 3], acc1);
  }
  return acc0 + acc1;
}

__device__ __forceinline__ float kq_dot(const Q6KRaw &raw, int g, const float (&x)[32]) {
#pragma clang fp contract(off)
  const int n0 = 32 * (g & 7);
  const int lo_sh = n0 < 128 ? 0 : 4;
  const int r = n0 >> 6;
  const int hi_sh = r == 0 ? 0 : (r == 1 ? 4 : (r == 2 ? 2 : 6));
  const float d = half_bits(raw.dh);
  const float ds0 = d * (float)(int)(signed char)(raw.sc2 & 0xFF);
  const float ds1 = d * (float)(int)(signed char)(raw.sc2 >> 8);
  const u4 ql[2] = {raw.ql0, raw.ql1}, qh[2] = {raw.qh0, raw.qh1};
  float acc[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const unsigned q = ((ql[i >> 2][i & 3] >> lo_sh) & 0x0F0F0F0Fu) |
                       (((qh[i >> 2][i & 3] >> hi_sh) & 0x03030303u) << 4);
    float(&a)[2] = acc[i >> 2];
    a[0] = __builtin_fmaf(ubyte_f32<0>(q) - 32.0f, x[4 * i], a[0]);
    a[1] = __builtin_fmaf(ubyte_f32<1>(q) - 32.0f, x[4 * i + 1], a[1]);
    a[0] = __builtin_fmaf(ubyte_f32<2>(q) - 32.0f, x[4 * i + 2], a[0]);
    a[1] = __builtin_fmaf(ubyte_f32<3>(q) - 32.0f, x[4 * i + 3], a[1]);
  }
  return ds0 * (acc[0][0] + acc[0][1]) + ds1 * (acc[1][0] + acc[1][1]);
}

// Q8_0 inputs (x = d_x * q_x per 32-value block, the group): the same
// weights against the integers q_x, the block's sum scaled by d_x once.
//   Q6_K: the sub-block sums sum (q - 32) q_x are exact integers (v_dot4 on
//         the 6-bit values, minus 32 sum q_x), then (ds0 S0 + ds1 S1) d_x.
//   Q4_K: the fp16 weights (formed as above) against q_x as fp16 (exact), two
//         products per v_dot2_f32_f16 (each product exact in fp32), then d_x.
// Both are the reference's sum of w * (d_x q_x) reassociated.
struct Q8Ints {   // one block: q_x as int8 and its two 16-value sums
  unsigned q[8];
  int s0, s1;
  float d;
};
struct Q8Halves {  // one block: q_x as fp16, values {4i, 4i + 2} and {4i + 1, 4i + 3}
  h2 a[8], b[8];
  float d;
};

__device__ __forceinline__ int sdot4(unsigned a, unsigned b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// 36-byte Q8_0 block -> both forms (the int8 and the fp16 values)
__device__ __forceinline__ void q8_ints(const unsigned (&blk)[9], Q8Ints &x) {
  x.d = __builtin_bit_cast(float, blk[0]);
  x.s0 = 0;
  x.s1 = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    x.q[i] = blk[1 + i];
    if (i < 4)
      x.s0 = sdot4(x.q[i], 0x01010101u, x.s0);
    else
      x.s1 = sdot4(x.q[i], 0x01010101u, x.s1);
  }
}

// four int8 -> fp16 pairs {q0, q2}, {q1, q3}: 1024 + (q + 128) by the 0x6400
// exponent, minus 1152 (all exact)
__device__ __forceinline__ void i8x4_halves(unsigned q, h2 &a, h2 &b) {
  const unsigned t = q ^ 0x80808080u;
  unsigned ua, ub;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(ua) : "v"(t), "s"(0x00FF00FFu), "v"(0x64006400u));
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(ub) : "v"(t >> 8), "s"(0x00FF00FFu), "v"(0x64006400u));
  const h2 k = {(_Float16)1152.0f, (_Float16)1152.0f};
  a = __builtin_bit_cast(h2, ua) - k;
  b = __builtin_bit_cast(h2, ub) - k;
}

__device__ __forceinline__ void q8_halves(const unsigned (&blk)[9], Q8Halves &x) {
  x.d = __builtin_bit_cast(float, blk[0]);
#pragma unroll
  for (int i = 0; i < 8; ++i) i8x4_halves(blk[1 + i], x.a[i], x.b[i]);
}

__device__ __forceinline__ float kq_dot8(const Q6KRaw &raw, int g, const Q8Ints &x) {
#pragma clang fp contract(off)
  const int n0 = 32 * (g & 7);
  const int lo_sh = n0 < 128 ? 0 : 4;
  const int r = n0 >> 6;
  const int hi_sh = r == 0 ? 0 : (r == 1 ? 4 : (r == 2 ? 2 : 6));
  const float d = half_bits(raw.dh);
  const float ds0 = d * (float)(int)(signed char)(raw.sc2 & 0xFF);
  const float ds1 = d * (float)(int)(signed char)(raw.sc2 >> 8);
  const u4 ql[2] = {raw.ql0, raw.ql1}, qh[2] = {raw.qh0, raw.qh1};
  int s0 = -32 * x.s0, s1 = -32 * x.s1;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const unsigned q = ((ql[i >> 2][i & 3] >> lo_sh) & 0x0F0F0F0Fu) |
                       (((qh[i >> 2][i & 3] >> hi_sh) & 0x03030303u) << 4);
    if (i < 4)
      s0 = sdot4(q, x.q[i], s0);
    else
      s1 = sdot4(q, x.q[i], s1);
  }
  return (ds0 * (float)s0 + ds1 * (float)s1) * x.d;
}

__device__ __forceinline__ float kq_dot8(const Q4KRaw &raw, int g, const Q8Halves &x) {
#pragma clang fp contract(off)
  const int j = g & 7;
  const u4 hdr = raw.hdr;
  const float d = half_bits(hdr[0] & 0xFFFF), dmin = half_bits(hdr[0] >> 16);
  const int p8 = 8 * (j & 3);
  const unsigned x1 = hdr[1] >> p8, x2 = hdr[2] >> p8, x3 = hdr[3] >> p8;
  const unsigned sv = j < 4 ? (x1 & 63) : ((x3 & 0xF) | ((x1 >> 2) & 0x30));
  const unsigned mv = j < 4 ? (x2 & 63) : (((x3 >> 4) & 0xF) | ((x2 >> 2) & 0x30));
  const _Float16 vd = (_Float16)(d * (float)sv), vm = (_Float16)(dmin * (float)mv);
  const h2 vd2 = {vd, vd}, vm2 = {vm, vm};
  const _Float16 c = (_Float16)-1024.0f * vd;
  const h2 c2 = {c, c}, k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
  const int sh = 4 * (j & 1);
  const unsigned magic = 0x64006400u;
  const bool fast = __all(__builtin_fabsf((float)vd) <= 63.5f);
  const u4 qv[2] = {raw.qa, raw.qb};
  float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const unsigned t = qv[i >> 2][i & 3] >> sh;
    unsigned ua, ub;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(ua) : "v"(t), "s"(0x000F000Fu), "v"(magic));
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(ub) : "v"(t >> 8), "s"(0x000F000Fu), "v"(magic));
    const h2 na = __builtin_bit_cast(h2, ua), nb = __builtin_bit_cast(h2, ub);
    h2 pa, pb;
    if (fast) {
      pa = __builtin_elementwise_fma(na, vd2, c2);
      pb = __builtin_elementwise_fma(nb, vd2, c2);
    } else {
      pa = (na - k1024) * vd2;
      pb = (nb - k1024) * vd2;
    }
    const h2 wa = pa - vm2, wb = pb - vm2;
    acc0 = __builtin_amdgcn_fdot2(wa, x.a[i], acc0, false);
    acc1 = __builtin_amdgcn_fdot2(wb, x.b[i], acc1, false);
  }
  return (acc0 + acc1) * x.d;
}

template <int TYPE>
using KqRaw = typename std::conditional<TYPE == kTypeQ4K, Q4KRaw, Q6KRaw>::type;
template <int TYPE>
using Q8Form = typename std::conditional<TYPE == kTypeQ4K, Q8Halves, Q8Ints>::type;

// Group pairs that share their quant bytes, one load for both: pair p of a
// row is groups g0 = 2p and 2p + 1 for Q4_K (a qs run's low and high
// nibbles) and g0 = 8 (p / 4) + p % 4 and g0 + 4 for Q6_K (the same ql and
// qh bytes; only the scales differ).
struct Q6KPair {
  u4 ql0, ql1, qh0, qh1;
  unsigned sc_a, sc_b, dh;
};
template <int TYPE>
using KqPair = typename std::conditional<TYPE == kTypeQ4K, Q4KRaw, Q6KPair>::type;

template <int TYPE>
__device__ __forceinline__ int pair_g0(int p) {
  return TYPE == kTypeQ4K ? 2 * p : 8 * (p >> 2) + (p & 3);
}
template <int TYPE>
__device__ __forceinline__ int pair_g1(int g0) {
  return TYPE == kTypeQ4K ? g0 + 1 : g0 + 4;
}

__device__ __forceinline__ void kq_load_pair(const uint8_t *row, int p, Q4KRaw &r) {
  kq_load(row, 2 * p, r);
}

__device__ __forceinline__ void kq_load_pair(const uint8_t *row, int p, Q6KPair &r) {
  const uint8_t *blk = row + (size_t)(p >> 2) * kQ6KBytes;
  const int n0 = 32 * (p & 3);
  r.ql0 = load_u4_unaligned(blk + n0);
  r.ql1 = load_u4_unaligned(blk + n0 + 16);
  r.qh0 = load_u4_unaligned(blk + 128 + (n0 & 63));
  r.qh1 = load_u4_unaligned(blk + 128 + (n0 & 63) + 16);
  r.sc_a = load_u16(blk + 192 + (n0 >> 4));
  r.sc_b = load_u16(blk + 200 + (n0 >> 4));
  r.dh = load_u16(blk + 208);
}

// pair p's two group sums, the first group's added first
template <int TYPE>
__device__ __forceinline__ void kq_dot8_pair(const KqPair<TYPE> &raw, int g0,
                                             const Q8Form<TYPE> &x0, const Q8Form<TYPE> &x1,
                                             float &acc) {
  if constexpr (TYPE == kTypeQ4K) {
    acc += kq_dot8(raw, g0, x0);
    acc += kq_dot8(raw, g0 + 1, x1);
  } else {
    Q6KRaw v;
    v.ql0 = raw.ql0;
    v.ql1 = raw.ql1;
    v.qh0 = raw.qh0;
    v.qh1 = raw.qh1;
    v.dh = raw.dh;
    v.sc2 = raw.sc_a;
    acc += kq_dot8(v, g0, x0);
    v.sc2 = raw.sc_b;
    acc += kq_dot8(v, g0 + 4, x1);
  }
}

template <int TYPE>
__device__ __forceinline__ void q8_form(const unsigned (&blk)[9], Q8Form<TYPE> &x) {
  if constexpr (TYPE == kTypeQ4K)
    q8_halves(blk, x);
  else
    q8_ints(blk, x);
}

// R rows per wave, 4 waves per workgroup.
template <int TYPE, bool XQ8, int R>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(XQ8 ? 4 : 1)))
kquant_matvec_kernel(const uint8_t *W, long row_bytes,
                                                            const void *x, float *y, int rows,
                                                            int cols) {
  const int lane = threadIdx.x & 63;
  const int row0 = (blockIdx.x * 4 + (threadIdx.x >> 6)) * R;
  if (row0 >= rows) return;  // whole wave
  const int ngroups = cols >> 5;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = 0.f;
  if constexpr (XQ8) {
    // Q8_0 blocks (fp32 d, 32 int8; 4-byte aligned), the reference's values
    // d * q (mistral_model.h:662-666) as d times the integers; a lane takes
    // group pairs
    const int npairs = ngroups >> 1;
    for (int p = lane; p < npairs; p += 64) {
      KqPair<TYPE> raw[R];
#pragma unroll
      for (int r = 0; r < R; ++r)  // a row past the end reloads the last row
        kq_load_pair(W + (size_t)min(row0 + r, rows - 1) * row_bytes, p, raw[r]);
      const int g0 = pair_g0<TYPE>(p), g1 = pair_g1<TYPE>(g0);
      const unsigned *b0 = reinterpret_cast<const unsigned *>(
          reinterpret_cast<const uint8_t *>(x) + (size_t)g0 * 36);
      const unsigned *b1 = reinterpret_cast<const unsigned *>(
          reinterpret_cast<const uint8_t *>(x) + (size_t)g1 * 36);
      unsigned w0[9], w1[9];
#pragma unroll
      for (int k = 0; k < 9; ++k) {
        w0[k] = b0[k];
        w1[k] = b1[k];
      }
      Q8Form<TYPE> x0, x1;
      q8_form<TYPE>(w0, x0);
      q8_form<TYPE>(w1, x1);
#pragma unroll
      for (int r = 0; r < R; ++r) kq_dot8_pair<TYPE>(raw[r], g0, x0, x1, acc[r]);
    }
  } else {
    for (int g = lane; g < ngroups; g += 64) {
      KqRaw<TYPE> raw[R];
#pragma unroll
      for (int r = 0; r < R; ++r)  // a row past the end reloads the last row
        kq_load(W + (size_t)min(row0 + r, rows - 1) * row_bytes, g, raw[r]);
      float xs[32];
      const f4 *xv = reinterpret_cast<const f4 *>(reinterpret_cast<const float *>(x) + 32 * g);
      f4 v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = xv[k];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        xs[4 * k] = v[k].x;
        xs[4 * k + 1] = v[k].y;
        xs[4 * k + 2] = v[k].z;
        xs[4 * k + 3] = v[k].w;
      }
#pragma unroll
      for (int r = 0; r < R; ++r) acc[r] += kq_dot(raw[r], g, xs);
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float v = wave_sum(acc[r]);
    if (lane == 0 && row0 + r < rows) y[row0 + r] = v;
  }
}

// The decode layer's K-quant matvecs (KqLayerParams): every workgroup of 8
// waves forms the Q8_0 blocks of its input in LDS while its first weight
// groups are in flight, then runs kquant_matvec_kernel<TYPE, true, R>'s loop
// on them.  Thread t loads the input's 4-value groups t + 512k, the groups of
// rmsnorm_kernel's thread t, so its sum of squares, the wave sums and their
// fixed combination are rmsnorm_kernel's own.  A workgroup's rows lie in one
// matrix.
template <int R, int XP, bool RMS>
__global__ void __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4)))
kq_layer_matvec_kernel(KqLayerParams p) {
#pragma clang fp contract(off)
  // the input's Q8_0 blocks twice: as the blocks (Q6_K rows), and as the
  // fp16 pairs of Q8Halves (Q4_K rows; group g's 16-byte chunk c at 4g +
  // ((c + g + g / 4) & 3), so that a wave's reads of a chunk are
  // conflict-free) with the scales apart
  __shared__ __attribute__((aligned(16))) uint8_t xq_lds[XP * 64 * 36];
  __shared__ u4 xh_lds[XP * 64 * 4];
  __shared__ float xd_lds[XP * 64];
  __shared__ float red[8];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rows01 = p.rows[0] + p.rows[1];
  const int total = rows01 + p.rows[2];
  const int row0 = (blockIdx.x * 8 + wave) * R;
  const int wg_row = blockIdx.x * 8 * R;
  const int m = wg_row < p.rows[0] ? 0 : (wg_row < rows01 ? 1 : 2);
  const int ngroups = p.cols >> 5;

  f4 xr[XP], ar[RMS ? XP : 1];
#pragma unroll
  for (int k = 0; k < XP; ++k) {
    const int blk = min(64 * k + (tid >> 3), ngroups - 1);
    const size_t off = (size_t)blk * 32 + (tid & 7) * 4;
    xr[k] = *reinterpret_cast<const f4 *>(p.xf + off);
    if constexpr (RMS) ar[k] = *reinterpret_cast<const f4 *>(p.rms_w + off);
  }
  __builtin_amdgcn_sched_barrier(0);

  auto prologue = [&]() {
#pragma clang fp contract(off)
    if constexpr (RMS) {
      // rmsnorm_vec (mistral_model.h:202-208) of the whole input
      float ss = 0.0f;
#pragma unroll
      for (int k = 0; k < XP; ++k) {
        const f4 v = xr[k];
        if (64 * k + (tid >> 3) < ngroups) ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
      }
      ss = wave_sum(ss);
      if (lane == 0) red[wave] = ss;
      // LDS writes visible; the weight loads stay outstanding
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      ss = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
      const float scale = 1.0f / sqrtf(ss / (float)p.cols + p.eps);
#pragma unroll
      for (int k = 0; k < XP; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) xr[k][e] = (xr[k][e] * scale) * ar[k][e];
    }
#pragma unroll
    for (int k = 0; k < XP; ++k) {
      const int blk = 64 * k + (tid >> 3);
      if (blk < ngroups) {  // whole 8-lane groups
        const int sub = tid & 7;
        f4 q;
        const float d = q8_block_q(xr[k], q);
        if (sub == 0) {
          *reinterpret_cast<float *>(xq_lds + blk * 36) = d;
          xd_lds[blk] = d;
        }
        *reinterpret_cast<unsigned *>(xq_lds + blk * 36 + 4 + 4 * sub) = q8_pack(q);
        const h2 a = {(_Float16)q[0], (_Float16)q[2]}, b = {(_Float16)q[1], (_Float16)q[3]};
        const int c = sub >> 1;
        u2 *dst = reinterpret_cast<u2 *>(&xh_lds[4 * blk + ((c + blk + (blk >> 2)) & 3)]);
        dst[sub & 1] = u2{__builtin_bit_cast(unsigned, a), __builtin_bit_cast(unsigned, b)};
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  };

  auto body = [&](auto type_tag) {
#pragma clang fp contract(off)
    constexpr int TYPE = decltype(type_tag)::value;
    const long rb = (long)(p.cols / kQKK) * (TYPE == kTypeQ4K ? kQ4KBytes : kQ6KBytes);
    const uint8_t *wrow[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {  // rows past the end reload the last row
      const int g = min(row0 + r, total - 1);
      const void *base;
      int lr;
      if (p.swiglu) {
        base = (g & 1) ? p.w[1] : p.w[0];
        lr = g >> 1;
      } else {
        base = p.w[m];
        lr = g - (m == 0 ? 0 : (m == 1 ? p.rows[0] : rows01));
      }
      wrow[r] = reinterpret_cast<const uint8_t *>(base) + (size_t)lr * rb;
    }
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    // the input's block g in the form the type's dot takes
    auto lds_form = [&](int g, Q8Form<TYPE> &xf) {
      if constexpr (TYPE == kTypeQ4K) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const u4 v = xh_lds[4 * g + ((c + g + (g >> 2)) & 3)];
          // each element through a scalar: __builtin_bit_cast of a vector
          // element (v.y ...) reads element 0 with this compiler
          const unsigned e0 = v.x, e1 = v.y, e2 = v.z, e3 = v.w;
          xf.a[2 * c] = __builtin_bit_cast(h2, e0);
          xf.b[2 * c] = __builtin_bit_cast(h2, e1);
          xf.a[2 * c + 1] = __builtin_bit_cast(h2, e2);
          xf.b[2 * c + 1] = __builtin_bit_cast(h2, e3);
        }
        xf.d = xd_lds[g];
      } else {
        const unsigned *blk = reinterpret_cast<const unsigned *>(xq_lds + g * 36);
        unsigned w[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) w[k] = blk[k];
        q8_ints(w, xf);
      }
    };
    const int npairs = ngroups >> 1;
    KqPair<TYPE> raw[R];
#pragma unroll
    for (int r = 0; r < R; ++r) kq_load_pair(wrow[r], min(lane, npairs - 1), raw[r]);
    __builtin_amdgcn_sched_barrier(0);
    prologue();
    for (int pp = lane; pp < npairs; pp += 64) {
      if (pp != lane) {
#pragma unroll
        for (int r = 0; r < R; ++r) kq_load_pair(wrow[r], pp, raw[r]);
      }
      const int g0 = pair_g0<TYPE>(pp), g1 = pair_g1<TYPE>(g0);
      Q8Form<TYPE> x0, x1;
      lds_form(g0, x0);
      lds_form(g1, x1);
#pragma unroll
      for (int r = 0; r < R; ++r) kq_dot8_pair<TYPE>(raw[r], g0, x0, x1, acc[r]);
    }
    float sum[R];
#pragma unroll
    for (int r = 0; r < R; ++r) sum[r] = wave_sum(acc[r]);
    if (p.swiglu) {
      // silu_mul_neon (mistral_model.h:174-199) of row j's gate and up sums
      if constexpr (R == 2) {
        if (lane == 0 && row0 < total) {
          const float gt = sum[0];
          const float sig = 1.0f / (1.0f + expf(-gt));
          p.y[0][row0 >> 1] = (gt * sig) * sum[1];
        }
      }
      return;
    }
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int g = row0 + r;
      if (lane == 0 && g < total) {
        const int mm = g < p.rows[0] ? 0 : (g < rows01 ? 1 : 2);
        float *y = p.y[mm] + (g - (mm == 0 ? 0 : (mm == 1 ? p.rows[0] : rows01)));
        *y = p.resid ? p.resid[g] + sum[r] : sum[r];
      }
    }
  };
  if (p.type[m] == kTypeQ4K)
    body(std::integral_constant<int, kTypeQ4K>{});
  else
    body(std::integral_constant<int, kTypeQ6K>{});
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

// The GEMM's fp16 operands, one workgroup per row.  Q4_K and F16 weights are
// fp16 values already: hi = w, no lo plane.  Q6_K and F32 weights are scaled by
// a power of two 2^e per row (the row's largest |w| lands in [2^13, 2^14), so
// that lo stays a normal fp16 for every weight within 2^-17 of the row's
// largest) and split, w 2^e = hi + lo to 2^-22 relative; rscale[row] = 2^-e.
template <int TYPE>
__global__ void __launch_bounds__(256) typed_f16_kernel(const uint8_t *W, long row_bytes,
                                                        _Float16 *hi, int rows, int cols) {
  const int ngroups = cols >> 5;
  const long total = (long)rows * ngroups;
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    const int r = (int)(i / ngroups), g = (int)(i % ngroups);
    float v[32];
    dequant_group<TYPE>(W + (size_t)r * row_bytes, g, v);
    h8 h[4];
#pragma unroll
    for (int k = 0; k < 32; ++k) h[k >> 3][k & 7] = (_Float16)v[k];  // exact
    h8 *dh = reinterpret_cast<h8 *>(hi + (size_t)r * cols + 32 * g);
#pragma unroll
    for (int k = 0; k < 4; ++k) dh[k] = h[k];
  }
}

template <int TYPE, bool LO>
__global__ void __launch_bounds__(256) typed_split_kernel(const uint8_t *W, long row_bytes,
                                                          _Float16 *hi, _Float16 *lo,
                                                          float *rscale, int rows, int cols) {
  __shared__ float wmax[4];
  const int ngroups = cols >> 5;
  for (int r = blockIdx.x; r < rows; r += gridDim.x) {
    const uint8_t *wr = W + (size_t)r * row_bytes;
    float scale = 1.0f;
    if constexpr (LO) {
      float m = 0.f;
      for (int g = threadIdx.x; g < ngroups; g += 256) {
        float v[32];
        dequant_group<TYPE>(wr, g, v);
#pragma unroll
        for (int l = 0; l < 32; ++l) m = fmaxf(m, fabsf(v[l]));
      }
      m = wave_max(m);
      if ((threadIdx.x & 63) == 0) wmax[threadIdx.x >> 6] = m;
      __syncthreads();
      m = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
      __syncthreads();  // wmax is rewritten for the next row
      int ex = 0;
      if (m > 0.f && m <= 3.4e38f) (void)frexpf(m, &ex);
      const int e = min(max(14 - ex, -60), 60);
      scale = ldexpf(1.0f, e);
      if (threadIdx.x == 0) rscale[r] = ldexpf(1.0f, -e);
    }
    for (int g = threadIdx.x; g < ngroups; g += 256) {
      float v[32];
      dequant_group<TYPE>(wr, g, v);
      h8 h[4], l4[4];
#pragma unroll
      for (int k = 0; k < 32; ++k) {
        const float x = v[k] * scale;
        const _Float16 xh = (_Float16)x;
        h[k >> 3][k & 7] = xh;
        if constexpr (LO) l4[k >> 3][k & 7] = (_Float16)(x - (float)xh);
      }
      h8 *dh = reinterpret_cast<h8 *>(hi + (size_t)r * cols + 32 * g);
#pragma unroll
      for (int k = 0; k < 4; ++k) dh[k] = h[k];
      if constexpr (LO) {
        h8 *dl = reinterpret_cast<h8 *>(lo + (size_t)r * cols + 32 * g);
#pragma unroll
        for (int k = 0; k < 4; ++k) dl[k] = l4[k];
      }
    }
  }
}

// Y [S][N] (+)= rscale[n] * ((C1 [S][N] + C1 [S + s][N]) + C2 [S][N]): the
// hi-activation and lo-activation products of the hi weights, plus the lo
// weights' product (C2, rscale: null for fp16-valued weights).
__global__ void __launch_bounds__(256) hilo_combine_kernel(const float *C1, const float *C2,
                                                           const float *rscale, float *Y, int S,
                                                           int N, bool add) {
#pragma clang fp contract(off)
  const long total = (long)S * N;
  if ((N & 3) == 0) {  // four outputs per thread (16-byte aligned rows)
    const long t4 = total >> 2;
    for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < t4; i += (long)gridDim.x * 256) {
      f4 v = reinterpret_cast<const f4 *>(C1)[i] + reinterpret_cast<const f4 *>(C1 + total)[i];
      if (C2) v = (v + reinterpret_cast<const f4 *>(C2)[i]) *
                  reinterpret_cast<const f4 *>(rscale)[(4 * i) % N >> 2];
      f4 *y = reinterpret_cast<f4 *>(Y) + i;
      *y = add ? *y + v : v;
    }
    return;
  }
  for (long i = (long)blockIdx.x * 256 + threadIdx.x; i < total; i += (long)gridDim.x * 256) {
    float v = C1[i] + C1[total + i];
    if (C2) v = (v + C2[i]) * rscale[i % N];
    Y[i] = add ? Y[i] + v : v;
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

template <int TYPE, int R>
void launch_kq_r(const uint8_t *w, long rb, const void *x, bool xq8, float *y, int rows, int cols,
                 hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  const dim3 grid((rows + 4 * R - 1) / (4 * R)), block(256);
  if (xq8) {
    if constexpr (R <= 2)  // launch_kq_matvec_t takes 1 or 2 rows per wave for Q8_0 inputs
      hipExtLaunchKernelGGL((kquant_matvec_kernel<TYPE, true, R>), grid, block, 0, s, ev0, ev1,
                            0, w, rb, x, y, rows, cols);
  } else
    hipExtLaunchKernelGGL((kquant_matvec_kernel<TYPE, false, R>), grid, block, 0, s, ev0, ev1, 0,
                          w, rb, x, y, rows, cols);
}

// Rows per wave, measured on the Mistral shapes: one row per wave while the
// matrix is small (the most waves in flight), more rows once there are
// enough waves and the x loads (128 B per lane and row for fp32 x, 72 B per
// group pair for Q8_0 blocks) start to cost; Q6_K rows on Q8_0 inputs, whose
// pairs carry 70 bytes each, one row per wave at every size.
template <int TYPE>
hipError_t launch_kq_matvec_t(const void *W, long rb, const void *x, bool xq8, float *y,
                              int rows, int cols, hipStream_t s, hipEvent_t ev0, hipEvent_t ev1) {
  const uint8_t *w = reinterpret_cast<const uint8_t *>(W);
  const bool large = (long)rows * cols >= (32L << 20);
  const int R = xq8 ? (TYPE == kTypeQ4K && large ? 2 : 1) : (rows < 2048 ? 1 : (large ? 4 : 2));
  if (R == 4)
    launch_kq_r<TYPE, 4>(w, rb, x, xq8, y, rows, cols, s, ev0, ev1);
  else if (R == 2)
    launch_kq_r<TYPE, 2>(w, rb, x, xq8, y, rows, cols, s, ev0, ev1);
  else
    launch_kq_r<TYPE, 1>(w, rb, x, xq8, y, rows, cols, s, ev0, ev1);
  return hipGetLastError();
}

template <int R, bool RMS>
hipError_t launch_kq_layer_r(const KqLayerParams &p, int ngroups, hipStream_t s, hipEvent_t ev0,
                             hipEvent_t ev1) {
  const int total = p.rows[0] + p.rows[1] + p.rows[2];
  const dim3 grid((total + 8 * R - 1) / (8 * R)), block(512);
  if (ngroups <= 64)
    hipExtLaunchKernelGGL((kq_layer_matvec_kernel<R, 1, RMS>), grid, block, 0, s, ev0, ev1, 0, p);
  else if (ngroups <= 128)
    hipExtLaunchKernelGGL((kq_layer_matvec_kernel<R, 2, RMS>), grid, block, 0, s, ev0, ev1, 0, p);
  else if (ngroups <= 256)
    hipExtLaunchKernelGGL((kq_layer_matvec_kernel<R, 4, RMS>), grid, block, 0, s, ev0, ev1, 0, p);
  else
    hipExtLaunchKernelGGL((kq_layer_matvec_kernel<R, 8, RMS>), grid, block, 0, s, ev0, ev1, 0, p);
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
    case kTypeQ4K: return launch_kq_matvec_t<kTypeQ4K>(W, rb, x, x_q8, y, rows, cols, s, ev0, ev1);
    case kTypeQ6K: return launch_kq_matvec_t<kTypeQ6K>(W, rb, x, x_q8, y, rows, cols, s, ev0, ev1);
    case kTypeF16: return launch_matvec_t<kTypeF16>(W, rb, x, x_q8, y, rows, cols, s, ev0, ev1);
    case kTypeF32: return launch_matvec_t<kTypeF32>(W, rb, x, x_q8, y, rows, cols, s, ev0, ev1);
    case kTypeQ40: return launch_matvec_t<kTypeQ40>(W, rb, x, x_q8, y, rows, cols, s, ev0, ev1);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_kq_layer_matvec(const KqLayerParams &p, hipStream_t s, hipEvent_t ev0,
                                  hipEvent_t ev1) {
  if (p.cols <= 0 || p.cols % kQKK || p.cols > kKqLayerMaxCols || !p.xf) return hipErrorInvalidValue;
  const int nmat = p.swiglu ? 2 : 3;
  for (int i = 0; i < 3; ++i) {
    if (p.rows[i] < 0) return hipErrorInvalidValue;
    if (p.rows[i] == 0) continue;
    if (i >= nmat || !p.w[i] || (p.type[i] != kTypeQ4K && p.type[i] != kTypeQ6K))
      return hipErrorInvalidValue;
  }
  const int total = p.rows[0] + p.rows[1] + p.rows[2];
  if (total <= 0) return hipErrorInvalidValue;
  // rows per wave as launch_typed_matvec picks them for Q8_0 inputs; the
  // SwiGLU form holds a gate row and its up row per wave
  const bool large = (long)total * p.cols >= (32L << 20);
  bool all_q4k = true;
  for (int i = 0; i < 3; ++i) all_q4k = all_q4k && (p.rows[i] == 0 || p.type[i] == kTypeQ4K);
  const int R = p.swiglu ? 2 : (all_q4k && large ? 2 : 1);
  if (p.swiglu && (p.rows[0] != p.rows[1] || p.rows[2] || p.type[0] != p.type[1] || p.resid))
    return hipErrorInvalidValue;
  if (!p.swiglu && (p.rows[0] % (8 * R) || (p.rows[0] + p.rows[1]) % (8 * R)))
    return hipErrorInvalidValue;  // a workgroup would straddle two matrices
  const int ngroups = p.cols >> 5;
  if (R == 2)
    return p.rms_w ? launch_kq_layer_r<2, true>(p, ngroups, s, ev0, ev1)
                   : launch_kq_layer_r<2, false>(p, ngroups, s, ev0, ev1);
  return p.rms_w ? launch_kq_layer_r<1, true>(p, ngroups, s, ev0, ev1)
                 : launch_kq_layer_r<1, false>(p, ngroups, s, ev0, ev1);
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

template <int TYPE, bool LO>
hipError_t launch_split_t(const void *W, long rb, _Float16 *hi, _Float16 *lo, float *rscale,
                          int rows, int cols, hipStream_t s) {
  const uint8_t *w = reinterpret_cast<const uint8_t *>(W);
  if constexpr (LO) {
    const int blocks = rows < 16384 ? rows : 16384;
    hipLaunchKernelGGL((typed_split_kernel<TYPE, true>), dim3(blocks), dim3(256), 0, s, w, rb, hi,
                       lo, rscale, rows, cols);
  } else {
    const long total = (long)rows * (cols >> 5);
    long blocks = (total + 255) / 256;
    if (blocks > 16384) blocks = 16384;
    hipLaunchKernelGGL((typed_f16_kernel<TYPE>), dim3((unsigned)blocks), dim3(256), 0, s, w, rb,
                       hi, rows, cols);
  }
  return hipGetLastError();
}

bool typed_is_f16_exact(int type) { return type == kTypeQ4K || type == kTypeF16; }

hipError_t launch_typed_split(const void *W, int type, _Float16 *hi, _Float16 *lo, float *rscale,
                              int rows, int cols, hipStream_t s) {
  const long rb = typed_row_bytes(type, cols);
  if (rb == 0 || rows <= 0) return hipErrorInvalidValue;
  switch (type) {
    case kTypeQ4K: return launch_split_t<kTypeQ4K, false>(W, rb, hi, lo, rscale, rows, cols, s);
    case kTypeF16: return launch_split_t<kTypeF16, false>(W, rb, hi, lo, rscale, rows, cols, s);
    case kTypeQ6K: return launch_split_t<kTypeQ6K, true>(W, rb, hi, lo, rscale, rows, cols, s);
    case kTypeF32: return launch_split_t<kTypeF32, true>(W, rb, hi, lo, rscale, rows, cols, s);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_hilo_combine(const float *C1, const float *C2, const float *rscale, float *Y,
                               int S, int N, bool add, hipStream_t s) {
  const long total = (long)S * N;
  long blocks = (total + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(hilo_combine_kernel, dim3((unsigned)blocks), dim3(256), 0, s, C1, C2, rscale,
                     Y, S, N, add);
  return hipGetLastError();
}

hipError_t launch_silu_mul(float *gate, const float *up, long n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  long blocks = (n + 255) / 256;
  if (blocks > 8192) blocks = 8192;
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)blocks), dim3(256), 0, s, gate, up, n);
  return hipGetLastError();
}

}  // namespace mia
