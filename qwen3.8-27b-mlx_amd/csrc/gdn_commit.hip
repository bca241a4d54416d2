// DeltaCache::commit(n) on the device (cpp/src/model.cpp:439-457): after a recorded
// (speculative) block of T steps, adopt the state after step n and the conv window
// rows n..n+2 of the padded conv input [conv_state_in ; x].
#include "gdn_internal.h"

namespace gdn {
namespace {

__global__ void commit_state_kernel(CommitParams p) {
  const size_t DD4 = (size_t)kD * kD / 4;
  const size_t heads = (size_t)p.n_layers * p.B * p.Hv;
  const size_t total = heads * DD4;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t head = i / DD4;  // (layer, b, h)
    const size_t e = i % DD4;
    const float4* src;
    if (p.n == 0) {
      src = reinterpret_cast<const float4*>(p.state_prev) + head * DD4;
    } else if (p.states_tbh) {
      const size_t h = head % p.Hv;
      const size_t lb = head / p.Hv;
      const size_t b = lb % p.B;
      const size_t layer = lb / p.B;
      src = reinterpret_cast<const float4*>(p.states) +
            ((((layer * p.T) + (p.n - 1)) * p.B + b) * p.Hv + h) * DD4;
    } else {
      src = reinterpret_cast<const float4*>(p.states) + (head * p.T + (p.n - 1)) * DD4;
    }
    reinterpret_cast<float4*>(p.state_dst)[head * DD4 + e] = src[e];
  }
}

// One thread per (layer, b, channel): reads the three source rows before writing, so
// the destination may be the conv state the block started from.
__global__ void commit_conv_kernel(CommitParams p) {
  const size_t total = (size_t)p.n_layers * p.B * p.C;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
       i += (size_t)gridDim.x * blockDim.x) {
    const size_t lb = i / p.C;
    const int c = (int)(i % p.C);
    const uint16_t* cin = p.conv_in ? p.conv_in + lb * kConvRows * p.C : nullptr;
    const uint16_t* x = p.x + lb * (size_t)p.T * p.C;
    uint16_t vals[kConvRows];
#pragma unroll
    for (int r = 0; r < kConvRows; ++r) {
      const int src = p.n + r;  // row of [conv_in ; x]
      if (src < kConvRows) {
        vals[r] = cin ? cin[(size_t)src * p.C + c] : (uint16_t)0;
      } else {
        vals[r] = x[(size_t)(src - kConvRows) * p.C + c];
      }
    }
    uint16_t* dst = p.conv_dst + lb * kConvRows * p.C;
#pragma unroll
    for (int r = 0; r < kConvRows; ++r) dst[(size_t)r * p.C + c] = vals[r];
  }
}

}  // namespace

hipError_t launch_commit(const CommitParams& p, hipStream_t stream) {
  // Nothing to copy when the destination already is the adopted state: n == 0 onto the
  // previous state, or the pointer swap (one layer, (T, B, Hv) states, destination = step
  // n-1's contiguous block).
  const bool keep_prev = p.n == 0 && p.state_prev == p.state_dst;
  const bool swapped = p.n > 0 && p.states_tbh && p.n_layers == 1 &&
                       p.states + (size_t)(p.n - 1) * p.B * p.Hv * kD * kD == p.state_dst;
  const bool copy_state = !keep_prev && !swapped;
  if (copy_state) {
    const size_t total = (size_t)p.n_layers * p.B * p.Hv * kD * kD / 4;
    const size_t blocks = std::min<size_t>((total + 255) / 256, 8192);
    if (blocks > 0) {
      hipLaunchKernelGGL(commit_state_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p);
      hipError_t e = hipGetLastError();
      if (e != hipSuccess) return e;
    }
  }
  if (p.C > 0 && p.conv_dst) {
    const size_t total = (size_t)p.n_layers * p.B * p.C;
    const size_t blocks = std::min<size_t>((total + 255) / 256, 4096);
    if (blocks > 0) {
      hipLaunchKernelGGL(commit_conv_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, p);
      return hipGetLastError();
    }
  }
  return hipSuccess;
}

}  // namespace gdn
