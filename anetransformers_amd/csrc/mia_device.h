// mia_device.h -- shared device-side helpers for the gfx950 attention kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace mia {

constexpr int HD = 128;  // head_dim the kernels are built for (mistral_model.h:404 fixes 128)

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));
typedef unsigned u2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

// log2(e) in fp32; the kernels fold it into the score scale and use exp2.
constexpr float kLog2e = 1.4426950408889634f;

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}

// All-reduce sum over each 16-lane DPP row: quad xor-1, quad xor-2, half-row
// mirror (lane i <-> 7-i), row mirror (lane i <-> 15-i).  Every lane of the
// row ends with the row sum.
__device__ __forceinline__ float row16_sum(float x) {
  x += dpp<0xB1>(x);   // quad_perm [1,0,3,2]
  x += dpp<0x4E>(x);   // quad_perm [2,3,0,1]
  x += dpp<0x141>(x);  // row_half_mirror
  x += dpp<0x140>(x);  // row_mirror
  return x;
}

__device__ __forceinline__ float row16_max(float x) {
  x = fmaxf(x, dpp<0xB1>(x));
  x = fmaxf(x, dpp<0x4E>(x));
  x = fmaxf(x, dpp<0x141>(x));
  x = fmaxf(x, dpp<0x140>(x));
  return x;
}

// Wave-wide (64 lanes) all-reduce: DPP within rows, then cross-row shuffles.
__device__ __forceinline__ float wave_sum(float x) {
  x = row16_sum(x);
  x += __shfl_xor(x, 16);
  x += __shfl_xor(x, 32);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
  x = row16_max(x);
  x = fmaxf(x, __shfl_xor(x, 16));
  x = fmaxf(x, __shfl_xor(x, 32));
  return x;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Keeps the compiler from moving LDS accesses across this point; LDS
// operations of one wave are executed in issue order by the hardware.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
  __builtin_amdgcn_wave_barrier();
}

// Adjacent-pair rotation of mistral/mistral_model.h:100-105 (vfmsq/vfmaq over
// a separately rounded vmulq): e' = fma(-o, s, e*c), o' = fma(e, s, o*c).
__device__ __forceinline__ void rope_pair(float &e, float &o, float c, float s) {
  float ec = e * c;
  float oc = o * c;
  float ne = __builtin_fmaf(-o, s, ec);
  float no = __builtin_fmaf(e, s, oc);
  e = ne;
  o = no;
}

// One Q8_0 block from an aligned group of 8 lanes holding 4 values each
// (values 4*sub .. 4*sub+3 of the block).  amax is order-free (max of absolute
// values), d = amax / 127 and id = 1 / d are IEEE-rounded divides, and
// q = round-half-even(x * id) saturated to int8, as vcvtnq_s32_f32 + vqmovn.
// Returns d; q holds this lane's 4 integers (as floats).
__device__ __forceinline__ float q8_block_q(const f4 v, f4 &q) {
  float a = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  a = fmaxf(a, __shfl_xor(a, 1));
  a = fmaxf(a, __shfl_xor(a, 2));
  a = fmaxf(a, __shfl_xor(a, 4));
  const float d = a / 127.0f;
  q = f4{0.0f, 0.0f, 0.0f, 0.0f};
  if (a != 0.0f) {
    const float id = 1.0f / d;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float r = __builtin_rintf(v[i] * id);
      q[i] = fminf(fmaxf(r, -128.0f), 127.0f);
    }
  }
  return d;
}

__device__ __forceinline__ unsigned q8_pack(const f4 q) {
  unsigned packed = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) packed |= ((unsigned)(int)q[i] & 0xFFu) << (8 * i);
  return packed;
}

// Writes d (lane sub 0) and this lane's 4 int8 to the 36-byte block at ob.
template <typename Byte>
__device__ __forceinline__ void q8_block_part(const f4 v, int sub, Byte *ob) {
  f4 q;
  const float d = q8_block_q(v, q);
  if (sub == 0) *reinterpret_cast<float *>(ob) = d;
  *reinterpret_cast<unsigned *>(ob + 4 + 4 * sub) = q8_pack(q);
}

}  // namespace mia
