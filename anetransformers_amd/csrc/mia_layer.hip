// mia_layer.hip -- the elementwise steps of the GPU decode layer
// (mistral_layer_decode_parallel, mistral/mistral_model.h:818-899) between
// its RMSNorms, projections and attention:
//   residual_rmsnorm_kernel  x += y (vDSP_vadd, :870), then out = rmsnorm_vec(x)
//                            (:873; mistral_model.h:202-208) in one launch
//   add_kernel               x += y (the FFN residual, :898)
// Both round as the reference: x + y once, sum of squares in fp32, scale =
// 1 / sqrtf(ss / dim + eps), out = (x * scale) * w.
#include "mia_device.h"
#include "mia_kernels.h"

namespace mia {

namespace {

// One workgroup of 512 threads, the sum order of rmsnorm_kernel; dim a
// multiple of 4, x / y / w / out 16-byte aligned.
__global__ __launch_bounds__(512) void residual_rmsnorm_kernel(float *x, const float *y,
                                                               const float *w, float *out,
                                                               int dim, float eps) {
#pragma clang fp contract(off)
  __shared__ float red[8];
  const int tid = threadIdx.x;
  float ss = 0.0f;
  for (int i = 4 * tid; i < dim; i += 4 * 512) {
    const f4 a = *reinterpret_cast<const f4 *>(x + i);
    const f4 b = *reinterpret_cast<const f4 *>(y + i);
    f4 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = a[e] + b[e];
    *reinterpret_cast<f4 *>(x + i) = v;
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  ss = ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
  const float scale = 1.0f / sqrtf(ss / (float)dim + eps);
  for (int i = 4 * tid; i < dim; i += 4 * 512) {  // the thread's own x values
    const f4 v = *reinterpret_cast<const f4 *>(x + i);
    const f4 wv = *reinterpret_cast<const f4 *>(w + i);
    f4 r;
#pragma unroll
    for (int e = 0; e < 4; ++e) r[e] = (v[e] * scale) * wv[e];
    *reinterpret_cast<f4 *>(out + i) = r;
  }
}

__global__ __launch_bounds__(256) void add_kernel(float *x, const float *y, int n) {
#pragma clang fp contract(off)
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n; i += gridDim.x * 256) x[i] = x[i] + y[i];
}

}  // namespace

hipError_t launch_residual_rmsnorm(float *x, const float *y, const float *w, float *out, int dim,
                                   float eps, hipStream_t s) {
  hipLaunchKernelGGL(residual_rmsnorm_kernel, dim3(1), dim3(512), 0, s, x, y, w, out, dim, eps);
  return hipGetLastError();
}

hipError_t launch_add(float *x, const float *y, int n, hipStream_t s) {
  if (n <= 0) return hipSuccess;
  const int blocks = (n + 255) / 256 < 1024 ? (n + 255) / 256 : 1024;
  hipLaunchKernelGGL(add_kernel, dim3(blocks), dim3(256), 0, s, x, y, n);
  return hipGetLastError();
}

}  // namespace mia
