// Memory streams with the shapes of the decode and verify state traffic, for bench.py's
// ceiling lines (libstream_probe.so, built by bench.py's build_probe(); not part of libgdn
// and not built by the package). They move the same bytes in the
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

// The decode step's full bytes: rmw_tile_kernel's tile plus each workgroup's share of the
// front end's traffic -- `fe_rd` float4 read from one buffer (x, conv state, conv weights,
// gate inputs) and `fe_wr` float4 written to another (conv state hand-off, o), issued as the
// kernel issues them: the front-end loads before the state loads, the writes last.
__global__ __launch_bounds__(256) void rmw_fe_kernel(f4* buf, int64_t per, const f4* fe_in, f4* fe_out, int fe_rd,
                                                     int fe_wr, float a, int group) {
  const int tile = tile_of_block(0, group);
  f4* base = buf + (int64_t)tile * per;
  const f4 fin = threadIdx.x < fe_rd ? fe_in[(int64_t)tile * fe_rd + threadIdx.x] : f4{0.f, 0.f, 0.f, 0.f};
  const int64_t per_thread = per / 256;
  f4 v[8];
  for (int64_t i0 = 0; i0 < per_thread; i0 += 8) {
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __builtin_nontemporal_load(base + (i0 + j) * 256 + threadIdx.x);
#pragma unroll
    for (int j = 0; j < 8; ++j) __builtin_nontemporal_store(v[j] * a, base + (i0 + j) * 256 + threadIdx.x);
  }
  if (threadIdx.x < fe_wr) fe_out[(int64_t)tile * fe_wr + threadIdx.x] = fin * a;
}

// Read-only: each workgroup reads its 32 KB tile (non-temporal); one float of the sum is
// stored only when it equals a value the data never holds, so the loads stay live.
__global__ __launch_bounds__(256) void read_tile_kernel(const f4* buf, float* sink) {
  const f4* base = buf + (int64_t)blockIdx.x * 2048;
  f4 v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = __builtin_nontemporal_load(base + j * 256 + threadIdx.x);
  f4 s = v[0];
#pragma unroll
  for (int j = 1; j < 8; ++j) s += v[j];
  if (s[0] + s[1] + s[2] + s[3] == -1.2345e38f) sink[0] = s[0];
}

// Write-only: each workgroup writes its 32 KB tile (plain stores: the fastest flavour for a
// write stream here).
__global__ __launch_bounds__(256) void write_tile_kernel(f4* buf, float a) {
  f4* base = buf + (int64_t)blockIdx.x * 2048;
#pragma unroll
  for (int j = 0; j < 8; ++j) base[j * 256 + threadIdx.x] = f4{a, a, a, (float)j};
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

// buf: tiles x 32 KB; fe_in: tiles x fe_rd float4; fe_out: tiles x fe_wr float4 (fe_rd,
// fe_wr <= 256); groups of `group` tiles per XCD turn (tiles % (8 group) == 0).
extern "C" int gdn_probe_rmw_fe(void* buf, const void* fe_in, void* fe_out, int tiles, int fe_rd, int fe_wr, int group,
                                void* stream) {
  if (!buf || !fe_in || !fe_out || fe_rd < 0 || fe_rd > 256 || fe_wr < 0 || fe_wr > 256 || group < 1 ||
      tiles < 8 * group || tiles % (8 * group))
    return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(rmw_fe_kernel, dim3(tiles), dim3(256), 0, (hipStream_t)stream, (f4*)buf, (int64_t)2048,
                     (const f4*)fe_in, (f4*)fe_out, fe_rd, fe_wr, 1.0001f, group);
  return (int)hipGetLastError();
}

// buf: tiles x 32 KB; sink: one float.
extern "C" int gdn_probe_read(const void* buf, void* sink, int tiles, void* stream) {
  if (!buf || !sink || tiles < 1) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(read_tile_kernel, dim3(tiles), dim3(256), 0, (hipStream_t)stream, (const f4*)buf, (float*)sink);
  return (int)hipGetLastError();
}

// buf: tiles x 32 KB.
extern "C" int gdn_probe_write(void* buf, int tiles, void* stream) {
  if (!buf || tiles < 1) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(write_tile_kernel, dim3(tiles), dim3(256), 0, (hipStream_t)stream, (f4*)buf, 1.0001f);
  return (int)hipGetLastError();
}

// src: tiles x 32 KB; dst: tiles x T x 32 KB.
extern "C" int gdn_probe_read_write_t(const void* src, void* dst, int tiles, int T, void* stream) {
  if (!src || !dst || tiles < 1 || T < 1) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(read_write_t_kernel, dim3(tiles), dim3(256), 0, (hipStream_t)stream, (const f4*)src, (f4*)dst, T,
                     1.0001f);
  return (int)hipGetLastError();
}
