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

}  // namespace mia
