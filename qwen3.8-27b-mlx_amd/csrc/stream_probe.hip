// Memory streams with the shapes of the decode and verify state traffic, for bench.py's
// ceiling lines (libgdn_probe.so; not part of libgdn's ABI). They move the same bytes in the
// same pattern as the kernels with none of the arithmetic, so the kernels' rate can be read
// against what this GPU streams for that pattern rather than only against the 8 TB/s peak.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

// Decode shape: each workgroup of 256 threads reads its 32 KB tile and writes it back in
// place (non-temporal both ways, as the decode state). Written as a loop over a run-time
// tile size: the compiler then stores each float4 as soon as its load has landed, which
// streams faster here (48.2 us for the decode step's 302 MB of state) than the same kernel
// with the size a constant, where it holds the stores back behind later loads (50.1 us).
// Workgroups are dispatched to the 8 XCDs round robin. split: each XCD takes one contiguous
// eighth of the tiles (the decode kernel's order for large grids); group > 0: groups of
// `group` consecutive tiles go to the XCDs in turn, dispatch id 8 group s + 8 j + x being
// tile j of group 8 s + x (its order for smaller grids).
__device__ __forceinline__ int tile_of_block(int split, int group) {
  int tile = (int)blockIdx.x;
  if (split) {
    tile = (int)((blockIdx.x & 7) * (gridDim.x >> 3) + (blockIdx.x >> 3));
  } else if (group > 0) {
    const int s = tile / (8 * group), r = tile % (8 * group);
    tile = group * (8 * s + (r & 7)) + (r >> 3);
  }
  return tile;
}

__global__ __launch_bounds__(256) void rmw_tile_kernel(f4* buf, int64_t per, float a, int split, int group) {
  f4* base = buf + (int64_t)tile_of_block(split, group) * per;
  const int64_t per_thread = per / 256;
  f4 v[8];
  for (int64_t i0 = 0; i0 < per_thread; i0 += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __builtin_nontemporal_load(base + (i0 + j) * 256 + threadIdx.x);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const f4 r = v[j] * a;
      __builtin_nontemporal_store(r, base + (i0 + j) * 256 + threadIdx.x);
    }
  }
}

// One-layer decode shape (16-row tiles of 8 KB, the decode kernel's grid for a single-layer
// call): each of the 256 threads reads two float4 and writes them back in place.
__global__ __launch_bounds__(256) void rmw_small_kernel(f4* buf, float a, int group) {
  f4* base = buf + (int64_t)tile_of_block(0, group) * 512;
  const f4 v0 = __builtin_nontemporal_load(base + threadIdx.x);
  const f4 v1 = __builtin_nontemporal_load(base + 256 + threadIdx.x);
  __builtin_nontemporal_store(v0 * a, base + threadIdx.x);
  __builtin_nontemporal_store(v1 * a, base + 256 + threadIdx.x);
}

// Verify shape: each workgroup reads its 32 KB tile and writes it T times (the per-step
// states), non-temporal.
__global__ __launch_bounds__(256) void read_write_t_kernel(const f4* src, f4* dst, int T, float a) {
  const f4* s = src + (int64_t)blockIdx.x * 2048;
  f4 v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = __builtin_nontemporal_load(s + j * 256 + threadIdx.x);
  for (int t = 0; t < T; ++t) {
    f4* d = dst + ((int64_t)blockIdx.x * T + t) * 2048;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[j] = v[j] * a;
      __builtin_nontemporal_store(v[j], d + j * 256 + threadIdx.x);
    }
  }
}

}  // namespace

// buf: tiles x 32 KB (16-byte aligned); returns a hipError_t.
extern "C" int gdn_probe_rmw(void* buf, int tiles, void* stream) {
  if (!buf || tiles < 1) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(rmw_tile_kernel, dim3(tiles), dim3(256), 0, (hipStream_t)stream, (f4*)buf, (int64_t)2048, 1.0001f, 0, 0);
  return (int)hipGetLastError();
}

// The same in groups of `group` consecutive tiles per XCD turn (tiles % (8 group) == 0).
extern "C" int gdn_probe_rmw_groups(void* buf, int tiles, int group, void* stream) {
  if (!buf || group < 1 || tiles < 8 * group || tiles % (8 * group)) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(rmw_tile_kernel, dim3(tiles), dim3(256), 0, (hipStream_t)stream, (f4*)buf, (int64_t)2048, 1.0001f, 0,
                     group);
  return (int)hipGetLastError();
}

// The same with each XCD streaming one contiguous eighth of the tiles (tiles % 8 == 0).
extern "C" int gdn_probe_rmw_split(void* buf, int tiles, void* stream) {
  if (!buf || tiles < 8 || tiles % 8) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(rmw_tile_kernel, dim3(tiles), dim3(256), 0, (hipStream_t)stream, (f4*)buf, (int64_t)2048, 1.0001f, 1, 0);
  return (int)hipGetLastError();
}

// buf: tiles x 8 KB; groups of `group` consecutive tiles per XCD turn (tiles % (8 group) == 0).
extern "C" int gdn_probe_rmw_small(void* buf, int tiles, int group, void* stream) {
  if (!buf || group < 1 || tiles < 8 * group || tiles % (8 * group)) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(rmw_small_kernel, dim3(tiles), dim3(256), 0, (hipStream_t)stream, (f4*)buf, 1.0001f, group);
  return (int)hipGetLastError();
}

// src: tiles x 32 KB; dst: tiles x T x 32 KB.
extern "C" int gdn_probe_read_write_t(const void* src, void* dst, int tiles, int T, void* stream) {
  if (!src || !dst || tiles < 1 || T < 1) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(read_write_t_kernel, dim3(tiles), dim3(256), 0, (hipStream_t)stream, (const f4*)src, (f4*)dst, T,
                     1.0001f);
  return (int)hipGetLastError();
}
