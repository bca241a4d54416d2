// Test probe (not part of libgdn): runs the device math of gdn_device_math.h -- the
// front ends' batched SiLU and the l2norm's bf16 reciprocal square root -- on arrays, so
// the GPU tests can compare every bf16 input with the oracle bit for bit. Built with the
// library's own compiler flags by tests/cpp/build.py.
#include <hip/hip_runtime.h>

#include "gdn_device_math.h"

namespace {

// Thread i applies silu_bf_batch<8> to y[8 i .. 8 i + 7] (the batch width of the front
// ends: a batch takes the exact path as a whole when any of its values does).
__global__ void silu_batch_kernel(const float* y, float* out, int batches) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= batches) return;
  float v[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = y[8 * i + e];
  gdn::silu_bf_batch(v);
#pragma unroll
  for (int e = 0; e < 8; ++e) out[8 * i + e] = v[e];
}

__global__ void rsqrt_kernel(const float* d, float* out, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) out[i] = gdn::rsqrt_bf(d[i]);
}

}  // namespace

extern "C" {

// y, out: device arrays of 8 * batches floats. Returns a hipError_t.
int probe_silu_bf_batch(const float* y, float* out, int batches) {
  if (batches <= 0) return 0;
  hipLaunchKernelGGL(silu_batch_kernel, dim3((batches + 255) / 256), dim3(256), 0, 0, y, out, batches);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipDeviceSynchronize();
  return (int)e;
}

// d, out: device arrays of n floats. Returns a hipError_t.
int probe_rsqrt_bf(const float* d, float* out, int n) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(rsqrt_kernel, dim3((n + 255) / 256), dim3(256), 0, 0, d, out, n);
  hipError_t e = hipGetLastError();
  if (e == hipSuccess) e = hipDeviceSynchronize();
  return (int)e;
}

}  // extern "C"
