// Quantized linear for the DeltaNet layer's projections on gfx950: y = x W^T with W in
// the reference's 4-bit affine layout (cpp/src/model.cpp:356-372, mx::quantized_matmul
// with transpose = true, group 64; python/mlp_kernel.py:54-56): uint32 words of 8 values,
// value i in nibble i (low nibble first), element = nibble * scale + bias per group of
// 64, scales and biases bf16. Up to four matrices that read the same x run in one launch
// (in_proj_qkv, in_proj_z, in_proj_a, in_proj_b of one layer), and an optional prologue
// applies the layer's GatedRMSNorm (model.cpp:350-354) to the recurrence output before
// out_proj, so norm and projection are one launch.
//
// HBM-bound at decode (M = B * L rows of x, 1..4): every weight byte is read once.
// Mapping: a workgroup stages its operand in LDS, then each wave takes 4 output rows at a
// time, one per 16-lane DPP row; lane m of a row reads the row's 16-byte pieces m, m + 16,
// m + 32, ... (each 32 nibbles = half a group), so a load instruction reads 4 x 256
// contiguous bytes; the rows' scale and bias words come 16 bytes a lane, ahead of the
// weights, and reach the lanes that use them through the wave's LDS rows. A nibble v becomes the bf16 value 128 + v with one and-or
// ((w >> 4i) & 0x000F000F | 0x43004300 gives nibbles i and i + 4 of the word as two bf16),
// v_dot2 multiplies pairs by the operand staged in the same pair order, and scale and
// bias are applied once per half-group: sum x (q s + b) = s * sum x (128 + q) +
// (b - 128 s) * sum x. The row total is a DPP row sum; the result is rounded to bf16 once.
//
// More rows (verify blocks, batched decode) run on MFMA (v_mfma_f32_16x16x32_bf16) with the
// same arithmetic: qprep writes the operand once into the workspace in the MFMA fragment
// order (the norm prologue applied there, as above) together with each row's sum x per
// 64-value group, then in qgemm each lane's weight row gives B fragments straight from its
// nibble words and the operand fragments come from the workspace; per group
// acc = sum x (128 + q) (fp32, MFMA), then y += s * acc + (b - 128 s) * sum x. In qgemm a
// workgroup's 4 waves split K and add their partial sums in LDS at the end, so each wave
// reads a quarter of the operand; calls of many weight rows and one m group (up to 64 rows,
// e.g. 8 layers of in_proj at once) take qgemm_ns instead, whose workgroup of 256 weight rows
// reads the operand into LDS once for its four waves.
#include "../../include/gdn.h"
#include "gdn_device_math.h"
#include "gdn_internal.h"

#include <algorithm>
#include <mutex>

namespace gdn {
namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
// global-memory pointers: a plain pointer that passed through a struct can lose its
// address space and compile to flat loads, which also count against the LDS wait counter
typedef const u32x2 __attribute__((address_space(1))) g_u32x2;
typedef const uint16_t __attribute__((address_space(1))) g_u16;

constexpr int kThreads = 256;
constexpr int kRowsPerPass = 16;  // 4 waves x 4 DPP rows

struct QParams {
  int M, K, R, tiles, nseg;
  int passes;            // row passes per workgroup: a tile is 16 x passes rows
  const uint16_t* x;     // (L, M, K) bf16, or NULL with the norm prologue
  const float* xf;       // (L, M, K) fp32 recurrence output (norm prologue)
  const uint16_t* z;     // (L, M, K) bf16 gate (norm prologue)
  const float* gamma;    // (L, 128) fp32 (norm prologue)
  float eps;
  const uint32_t* w[GDN_QLINEAR_MAX_SEGS];
  const uint16_t* s[GDN_QLINEAR_MAX_SEGS];
  const uint16_t* b[GDN_QLINEAR_MAX_SEGS];
  uint16_t* y[GDN_QLINEAR_MAX_SEGS];
  int n[GDN_QLINEAR_MAX_SEGS];
  int row0[GDN_QLINEAR_MAX_SEGS];  // first global row of each segment
  // MFMA path: the operand in fragment order, (L, mtiles, K / 32) blocks of 64 lanes x 8
  // bf16; lane 16 g4 + mm of block f = 2 g + s holds row 16 mt + mm, values
  // k = 64 g + 16 g4 + 8 s + (0, 4, 1, 5, 2, 6, 3, 7) (the nibble pair order); rows past M
  // are zeros
  uint16_t* xfrag;
  // MFMA path: sum x of each 64-value group, fp32, (L, K / 64, 16 mtiles): row-contiguous
  // per group, so a workgroup's m tiles of one group are one run
  float* xsum;
  int mtiles;
  int mgroups;  // MFMA path: groups of MT m-tiles (the grid is layers x tiles x mgroups)
  int remap;    // MFMA path: XCD-aware workgroup order (see qgemm_kernel)
};

__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf2, a), __builtin_bit_cast(bf2, b), c, false);
}

__device__ __forceinline__ uint32_t pack_bf2(float lo, float hi) {
  return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

// Operand chunk (32 values) to LDS: four 16-byte words, word i holding the pairs
// (v[8i+j], v[8i+j+4]), j = 0..3, the order the nibble pairs come out in; plus the sum
// of the 32 values.
__device__ __forceinline__ void stage_chunk(u32x4* xs, float* xsum, int nch, int mm, int c, const float (&v)[32]) {
  float sum = 0.0f;
#pragma unroll
  for (int e = 0; e < 32; ++e) sum += v[e];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    u32x4 q;
#pragma unroll
    for (int j = 0; j < 4; ++j) q[j] = pack_bf2(v[8 * i + j], v[8 * i + j + 4]);
    xs[(mm * 4 + i) * nch + c] = q;
  }
  xsum[mm * nch + c] = sum;
}

// The operand of row mrow, values 32 c .. 32 c + 31, into v: x as given, or the GatedRMSNorm
// of (xf, z) (the four pieces of a 128-value head are the lanes of a DPP quad).
template <bool NORM>
__device__ __forceinline__ void operand_piece(const QParams& p, int layer, int mrow, int c, float (&v)[32]) {
  const size_t base = ((size_t)layer * p.M + mrow) * p.K + 32 * c;
  if (NORM) {
    // GatedRMSNorm: h = o * rsqrt(mean(o^2) + eps) * gamma (fp32), times silu(fp32(z)),
    // rounded to bf16 (the activation dtype out_proj takes)
    float o[32];
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const f4 f = *reinterpret_cast<const f4*>(p.xf + base + 4 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e) o[4 * q + e] = f[e];
    }
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 32; ++e) ss += o[e] * o[e];
    ss += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, ss), 0xB1, 0xF, 0xF, true));
    ss += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, ss), 0x4E, 0xF, 0xF, true));
    const float rs = 1.0f / sqrtf(ss / 128.0f + p.eps);
    const float* gm = p.gamma + (size_t)layer * 128 + 32 * (c & 3);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u16x8 zz = *reinterpret_cast<const u16x8*>(p.z + base + 8 * q);
      const f4 g0 = *reinterpret_cast<const f4*>(gm + 8 * q);
      const f4 g1 = *reinterpret_cast<const f4*>(gm + 8 * q + 4);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float zf = bf2f(zz[e]);
        const float h = o[8 * q + e] * rs * (e < 4 ? g0[e] : g1[e - 4]);
        v[8 * q + e] = rbf(h * (zf * d_sigmoidf(zf)));
      }
    }
  } else {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const u16x8 xx = *reinterpret_cast<const u16x8*>(p.x + base + 8 * q);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[8 * q + e] = bf2f(xx[e]);
    }
  }
}

// (a & m) | c: with m and c in VGPRs (opaque values from nibble_consts) the compiler selects
// one v_and_or_b32 for it -- with literal constants it cannot (a VOP3 takes no literal on
// this target and at most one SGPR) and emits a separate AND and OR. Written out in C, not
// as inline asm, so that the compiler also sees the instruction and keeps the wait states
// an MFMA reading its result needs.
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t m, uint32_t c) { return (a & m) | c; }
struct NibbleConsts {
  uint32_t mask, bias;  // 0x000F000F, 0x43004300
};
__device__ __forceinline__ NibbleConsts nibble_consts() {
  NibbleConsts k;
  k.mask = 0x000F000Fu;
  k.bias = 0x43004300u;
  asm volatile("" : "+v"(k.mask), "+v"(k.bias));  // (emits nothing: keeps them opaque VGPR values)
  return k;
}

template <int J, bool NORM>
__global__ __launch_bounds__(kThreads) void qlinear_kernel(QParams p) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  // each wave's scale and bias words of its current 4 rows: [wave][row][scale, bias][group]
  __shared__ __attribute__((aligned(16))) uint16_t sbs[4][4][2][8192 / 64];
  const int layer = blockIdx.x / p.tiles;
  const int tile = blockIdx.x % p.tiles;
  const int K = J * 512, nch = K / 32;
  u32x4* xs = reinterpret_cast<u32x4*>(smem);                 // [M][4][nch]
  float* xsum = reinterpret_cast<float*>(xs + p.M * 4 * nch);  // [M][nch]
  const int tid = threadIdx.x;

  // ---- stage the operand: thread task t = (row mm, chunk c); the four chunks of a
  // 128-value head are the four lanes of a DPP quad ----
  for (int t = tid; t < p.M * nch; t += kThreads) {
    const int mm = t / nch, c = t % nch;
    float v[32];
    operand_piece<NORM>(p, layer, mm, c, v);
    stage_chunk(xs, xsum, nch, mm, c, v);
  }
  __syncthreads();

  // ---- passes of 4 rows per wave ----
  const NibbleConsts nk = nibble_consts();
  const int lane = tid & 63, m = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int passes = p.passes;
  for (int pass = 0; pass < passes; ++pass) {
    const int grow = (tile * passes + pass) * kRowsPerPass + wave * 4 + (lane >> 4);
    const bool valid = grow < p.R;
    const int row = valid ? grow : p.R - 1;
    int sg = 0;
#pragma unroll
    for (int q = 1; q < GDN_QLINEAR_MAX_SEGS; ++q) sg += (q < p.nseg && row >= p.row0[q]) ? 1 : 0;
    const uint32_t* wseg = p.w[0];
    const uint16_t *sseg = p.s[0], *bseg = p.b[0];
    uint16_t* yseg = p.y[0];
    int nseg = p.n[0], r0 = p.row0[0];
#pragma unroll
    for (int q = 1; q < GDN_QLINEAR_MAX_SEGS; ++q) {
      if (sg == q) {
        wseg = p.w[q];
        sseg = p.s[q];
        bseg = p.b[q];
        yseg = p.y[q];
        nseg = p.n[q];
        r0 = p.row0[q];
      }
    }
    const size_t lrow = (size_t)layer * nseg + (row - r0);
    const u32x4* wr = reinterpret_cast<const u32x4*>(wseg + lrow * (K / 8));
    const uint16_t* sr = sseg + lrow * (K / 64);
    const uint16_t* br = bseg + lrow * (K / 64);
    // the row's scale and bias words, 16 bytes a lane (groups 8 mc .. + 7; lanes past the
    // row's K / 512 chunks repeat the last), first: they arrive before the weights
    const int mc = m < J ? m : J - 1;
    const u32x4 swd = *reinterpret_cast<const u32x4*>(sr + 8 * mc);
    const u32x4 bwd = *reinterpret_cast<const u32x4*>(br + 8 * mc);
    u32x4 wv[J];
#pragma unroll
    for (int j = 0; j < J; ++j) wv[j] = __builtin_nontemporal_load(wr + m + 16 * j);
    // through this wave's LDS rows (written and read by this wave only: no barrier) to the
    // lanes that use them: piece m + 16 j is in group m / 2 + 8 j
    uint16_t* srl = &sbs[wave][lane >> 4][0][0];
    uint16_t* brl = &sbs[wave][lane >> 4][1][0];
    *reinterpret_cast<u32x4*>(srl + 8 * mc) = swd;
    *reinterpret_cast<u32x4*>(brl + 8 * mc) = bwd;
    float y[GDN_QLINEAR_GEMV_ROWS] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < J; ++j) {
      const int c = m + 16 * j;
      const float sc = bf2f(srl[(m >> 1) + 8 * j]);
      const float off = bf2f(brl[(m >> 1) + 8 * j]) - 128.0f * sc;
      uint32_t pr[4][4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t wd = wv[j][i];
#pragma unroll
        for (int q = 0; q < 4; ++q) pr[i][q] = and_or(wd >> (4 * q), nk.mask, nk.bias);
      }
#pragma unroll
      for (int mm = 0; mm < GDN_QLINEAR_GEMV_ROWS; ++mm) {
        if (mm < p.M) {
          float acc = 0.0f;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const u32x4 xq = xs[(mm * 4 + i) * nch + c];
#pragma unroll
            for (int q = 0; q < 4; ++q) acc = dot2(pr[i][q], xq[q], acc);
          }
          y[mm] = __builtin_fmaf(sc, acc, __builtin_fmaf(off, xsum[mm * nch + c], y[mm]));
        }
      }
    }
#pragma unroll
    for (int mm = 0; mm < GDN_QLINEAR_GEMV_ROWS; ++mm) {
      if (mm < p.M) {
        const float tot = row16_sum(y[mm]);
        if (m == 0 && valid) yseg[((size_t)layer * p.M + mm) * nseg + (row - r0)] = f2bf(tot);
      }
    }
  }
}

// MFMA path, step 1: the operand (normalised when NORM) into the workspace's fragment
// order. Thread = (layer, row, 32-value piece c, quarter j): 8 consecutive values, one
// fragment lane (block 2 (c / 2) + j % 2, lane 16 (2 (c % 2) + j / 2) + row % 16), so four
// consecutive threads read a piece's contiguous bytes and a 16-lane DPP row holds one
// 128-value head (nch is a multiple of 4). For the norm, each thread sums its 8 squares and
// the row adds the 16 partial sums.
template <bool NORM>
__global__ __launch_bounds__(kThreads) void qprep_kernel(QParams p, int layers) {
  const int nch = p.K / 32, rows = 16 * p.mtiles;
  const size_t tt = (size_t)blockIdx.x * kThreads + threadIdx.x;
  if (tt >= (size_t)layers * rows * nch * 4) return;  // whole 16-lane rows
  const int j = (int)(tt & 3);
  const size_t t = tt >> 2;
  const int c = (int)(t % nch);
  const size_t rg = t / nch;
  const int mrow = (int)(rg % rows), layer = (int)(rg / rows);
  const bool live = mrow < p.M;
  const size_t base = ((size_t)layer * p.M + (live ? mrow : 0)) * p.K + 32 * c + 8 * j;
  float v[8];
  if (NORM) {
    // GatedRMSNorm (model.cpp:350-354): h = o * rsqrt(mean(o^2) + eps) * gamma (fp32), times
    // silu(fp32(z)), rounded to bf16 (the activation dtype out_proj takes)
    const f4 o0 = *reinterpret_cast<const f4*>(p.xf + base);
    const f4 o1 = *reinterpret_cast<const f4*>(p.xf + base + 4);
    const u16x8 zz = *reinterpret_cast<const u16x8*>(p.z + base);
    const float* gm = p.gamma + (size_t)layer * 128 + 32 * (c & 3) + 8 * j;
    const f4 g0 = *reinterpret_cast<const f4*>(gm);
    const f4 g1 = *reinterpret_cast<const f4*>(gm + 4);
    float ss = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += o0[e] * o0[e];
#pragma unroll
    for (int e = 0; e < 4; ++e) ss += o1[e] * o1[e];
    ss = row16_sum(ss);
    const float rs = 1.0f / sqrtf(ss / 128.0f + p.eps);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float zf = bf2f(zz[e]);
      const float h = (e < 4 ? o0[e] : o1[e - 4]) * rs * (e < 4 ? g0[e] : g1[e - 4]);
      v[e] = live ? rbf(h * (zf * d_sigmoidf(zf))) : 0.0f;
    }
  } else {
    const u16x8 xx = *reinterpret_cast<const u16x8*>(p.x + base);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = live ? bf2f(xx[e]) : 0.0f;
  }
  uint16_t* blk = p.xfrag + ((size_t)layer * p.mtiles + mrow / 16) * nch * 512;
  u32x4 q;
#pragma unroll
  for (int e = 0; e < 4; ++e) q[e] = pack_bf2(v[e], v[e + 4]);
  const int f = 2 * (c / 2) + (j & 1), ln = 16 * (2 * (c & 1) + j / 2) + (mrow & 15);
  *reinterpret_cast<u32x4*>(blk + ((size_t)f * 64 + ln) * 8) = q;
  // the group's sum x: the 64 values of (row, group c / 2) are the 8 values of each of 8
  // consecutive threads (pieces c, c + 1 of a group are adjacent: nch is even), added in
  // a fixed order (each thread's 8 in sequence, then a butterfly over the 8 threads)
  float sx = 0.0f;
#pragma unroll
  for (int e = 0; e < 8; ++e) sx += v[e];
  sx += __shfl_xor(sx, 1, 8);
  sx += __shfl_xor(sx, 2, 8);
  sx += __shfl_xor(sx, 4, 8);
  if ((tt & 7) == 0) p.xsum[((size_t)layer * (p.K / 64) + c / 2) * rows + mrow] = sx;
}

__device__ __forceinline__ f4 mfma(bf8 a, bf8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// A nibble word (values k .. k + 7) as a B fragment: bf16 128 + v, pairs (i, i + 4).
__device__ __forceinline__ bf8 nibbles_bf16(uint32_t wd, NibbleConsts k) {
  u32x4 r;
#pragma unroll
  for (int q = 0; q < 4; ++q) r[q] = and_or(wd >> (4 * q), k.mask, k.bias);
  return __builtin_bit_cast(bf8, r);
}

// A weight row's segment: its nibble words, scales, biases and output column. Every
// candidate is read as a value first and held opaque (the empty asm), then selected: a
// select between loads of the argument arrays is otherwise folded into one load at a
// run-time index, for which the compiler copies the kernel arguments to scratch.
struct RowPtrs {
  const uint32_t* w;
  const uint16_t *s, *b;
  uint16_t* y;
  int ystride;
};
__device__ __forceinline__ RowPtrs row_ptrs(const QParams& p, int layer, int row) {
  const uint32_t* wv[GDN_QLINEAR_MAX_SEGS];
  const uint16_t *sv[GDN_QLINEAR_MAX_SEGS], *bv[GDN_QLINEAR_MAX_SEGS];
  uint16_t* yv[GDN_QLINEAR_MAX_SEGS];
  int nv[GDN_QLINEAR_MAX_SEGS], rv[GDN_QLINEAR_MAX_SEGS];
#pragma unroll
  for (int q = 0; q < GDN_QLINEAR_MAX_SEGS; ++q) {
    wv[q] = p.w[q];
    sv[q] = p.s[q];
    bv[q] = p.b[q];
    yv[q] = p.y[q];
    nv[q] = p.n[q];
    rv[q] = p.row0[q];
    asm volatile("" : "+s"(wv[q]), "+s"(sv[q]), "+s"(bv[q]), "+s"(yv[q]), "+s"(nv[q]), "+s"(rv[q]));
  }
  int sg = 0;
#pragma unroll
  for (int q = 1; q < GDN_QLINEAR_MAX_SEGS; ++q) sg += (q < p.nseg && row >= rv[q]) ? 1 : 0;
  const uint32_t* wseg = wv[0];
  const uint16_t *sseg = sv[0], *bseg = bv[0];
  uint16_t* yseg = yv[0];
  int nseg = nv[0], r0 = rv[0];
#pragma unroll
  for (int q = 1; q < GDN_QLINEAR_MAX_SEGS; ++q) {
    if (sg == q) {
      wseg = wv[q];
      sseg = sv[q];
      bseg = bv[q];
      yseg = yv[q];
      nseg = nv[q];
      r0 = rv[q];
    }
  }
  const int G = p.K / 64;
  const size_t lrow = (size_t)layer * nseg + (row - r0);
  RowPtrs r;
  r.w = wseg + lrow * (p.K / 8);
  r.s = sseg + lrow * G;
  r.b = bseg + lrow * G;
  r.y = yseg + (size_t)layer * p.M * nseg + (row - r0);
  r.ystride = nseg;
  return r;
}

// MFMA path, step 2. Workgroup = 16 NT weight rows (the output columns) x 16 MT operand
// rows; wave w takes the groups g = 4 i + w, i < G / 4, of the G = K / 64 groups (a multiple
// of 4 for every supported K), so the four groups of a weight row's 128-byte line are asked
// for by the four waves together and the line is fetched once (when each wave took a
// contiguous quarter of K, a line's four groups were read at four different times and
// lines were fetched again after eviction). Lane (g4, nn) = (l / 16, l % 16) takes the
// nibble words 8 g + 2 g4 + s of its row 16 nt + nn (loaded by another lane, see below) and
// gets C rows m = 4 g4 + i of column nn.
// Memory: the weight stream comes from HBM once, so what bounds the kernel is how many of
// its bytes each wave keeps in flight: every load is issued kRing groups ahead (the ring
// below), and the workgroup's scale and bias pairs are staged in LDS once at the start
// (they would otherwise be two more loads per row tile and group at the same depth).
constexpr int kRing = 2;  // groups in flight per wave (G / 4 is a multiple of it)
template <int MT, int NT>
__global__ __launch_bounds__(kThreads) void qgemm_kernel(QParams p) {
  constexpr int kRows = 16 * NT;
  constexpr int kMaxG = 8192 / 64;
  // scale | bias << 16 per (row, group), rows kMaxG + 1 words apart at most (a row stride
  // of G + 1 words puts the 16 rows a wave reads at once on distinct banks); at the end the
  // partial sums of waves 1..3
  __shared__ __attribute__((aligned(16))) union {
    uint32_t sb[kRows * (kMaxG + 1)];
    f4 red[3][MT * NT][64];
  } sm;
  // the operand's group sums for this workgroup's MT m tiles, all groups: [group][16 MT]
  __shared__ __attribute__((aligned(16))) float xs_l[kMaxG * 16 * MT];
  // Workgroup = (layer, weight tile, m group), m groups fastest. Workgroups are dispatched to
  // the 8 XCDs round robin; the ids are renumbered (p.remap) so that each XCD runs a
  // contiguous range: with several m groups, all m groups of a weight tile on one XCD, one
  // after another, so its weight rows come from HBM once and from that XCD's L2 after; with
  // 8 layers or more, whole layers per XCD, so a layer's operand is read from HBM into one
  // L2 instead of all eight.
  int bid = blockIdx.x;
  if (p.remap) bid = (bid & 7) * (int)(gridDim.x >> 3) + (bid >> 3);
  const int mg = bid % p.mgroups, lt = bid / p.mgroups;
  const int layer = lt / p.tiles, tile = lt % p.tiles;
  const int mt0 = mg * MT;
  const int lane = threadIdx.x & 63, g4 = lane >> 4, nn = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = p.K, G = K / 64, nch = K / 32, sbs = G + 1;
  const int ng = G / 4;  // this wave's groups: 4 i + wave, i < ng

  // Weight loads are laid out for the memory path, not for the MFMA: lane 4 r + c reads the
  // 8-byte chunk c (words 2 c, 2 c + 1) of row r's group, so the 32 bytes of a row's group
  // come from one lane quad in one L1 access (with lane 16 c + r reading them, the four
  // lanes of every quad hit four rows: four times the L1 accesses, and the address path
  // saturates). The B fragment wants chunk g4 of row nn in lane 16 g4 + nn, so each loaded
  // word pair crosses lanes with ds_bpermute before its nibbles are expanded.
  const int bsrc = (4 * nn + g4) * 4;  // byte address of the lane that loaded (nn, g4)
  g_u32x2* wr[NT];
  uint16_t* yr[NT];
  int ystride[NT];
  bool valid[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int grow = (tile * NT + nt) * 16 + nn;
    valid[nt] = grow < p.R;
    const RowPtrs rp = row_ptrs(p, layer, valid[nt] ? grow : p.R - 1);
    yr[nt] = rp.y;
    ystride[nt] = rp.ystride;
    const int lrow = (tile * NT + nt) * 16 + (lane >> 2);
    const RowPtrs rl = row_ptrs(p, layer, lrow < p.R ? lrow : p.R - 1);
    wr[nt] = (g_u32x2*)(rl.w) + (lane & 3);  // + 4 g: words 8 g + 2 c, +1
  }
  const bf8* xa = reinterpret_cast<const bf8*>(p.xfrag + ((size_t)layer * p.mtiles + mt0) * nch * 512) + lane;
  const NibbleConsts nk = nibble_consts();

  // A ring of kRing slots, one group each (operand fragments and nibble words): slot j
  // holds groups j, j + kRing, ... and is reloaded with the group kRing ahead right after
  // its products, so every load is issued kRing groups before its use. (Loads complete in
  // issue order: a nearer load issued after a farther one would wait for it.) Loads past
  // the wave's last group reload that group, unused.
  struct Slot {
    bf8 a[MT][2];
    u32x2 w[NT];
  };
  auto load = [&](int g, Slot& sl) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int s = 0; s < 2; ++s) sl.a[mt][s] = xa[((size_t)mt * nch + 2 * g + s) * 64];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) sl.w[nt] = wr[nt][4 * g];
  };
  Slot R[kRing];
#pragma unroll
  for (int j = 0; j < kRing; ++j) load(4 * j + wave, R[j]);  // (ng >= kRing)

  // the scale and bias pairs of the workgroup's rows, all groups: thread t takes row
  // t / (256 / kRows), four groups at a time (8-byte loads: G and the block starts are
  // multiples of 4)
  {
    constexpr int tpr = kThreads / kRows;
    const int r = threadIdx.x / tpr, j = threadIdx.x % tpr;
    const int grow = tile * kRows + r;
    const RowPtrs rp = row_ptrs(p, layer, grow < p.R ? grow : p.R - 1);
    for (int g = 4 * j; g < G; g += 4 * tpr) {
      const u32x2 sv = *(g_u32x2*)(rp.s + g);
      const u32x2 bv = *(g_u32x2*)(rp.b + g);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t s16 = (sv[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
        const uint32_t b16 = (bv[e >> 1] >> (16 * (e & 1))) & 0xFFFFu;
        sm.sb[r * sbs + g + e] = s16 | (b16 << 16);
      }
    }
    // the group sums: 4 MT float4 per group, contiguous in xsum
    const float* xsg = p.xsum + (size_t)layer * G * (16 * p.mtiles) + 16 * mt0;
    for (int q = threadIdx.x; q < 4 * MT * G; q += kThreads) {
      const int g = q / (4 * MT), o = 4 * (q % (4 * MT));
      *reinterpret_cast<f4*>(&xs_l[g * 16 * MT + o]) = *reinterpret_cast<const f4*>(xsg + (size_t)g * 16 * p.mtiles + o);
    }
  }
  __syncthreads();

  f4 y[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) y[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};

  // the wave's i-th group from slot sl, then sl reloaded with its (i + kRing)-th
  auto step = [&](int i, Slot& sl) {
    const int g = 4 * i + wave;
    f4 xs[MT];  // sum x of the group for this lane's rows 4 g4 .. + 3 of each m tile
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xs[mt] = *reinterpret_cast<const f4*>(&xs_l[g * 16 * MT + 16 * mt + 4 * g4]);
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const uint32_t sbv = sm.sb[(16 * nt + nn) * sbs + g];
      const float sc = __builtin_bit_cast(float, sbv << 16);
      const float off = __builtin_bit_cast(float, sbv & 0xFFFF0000u) - 128.0f * sc;
      const uint32_t w0 = (uint32_t)__builtin_amdgcn_ds_bpermute(bsrc, (int)sl.w[nt][0]);
      const uint32_t w1 = (uint32_t)__builtin_amdgcn_ds_bpermute(bsrc, (int)sl.w[nt][1]);
      const bf8 b0 = nibbles_bf16(w0, nk), b1 = nibbles_bf16(w1, nk);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        f4 acc = mfma(sl.a[mt][0], b0, f4{0.f, 0.f, 0.f, 0.f});
        acc = mfma(sl.a[mt][1], b1, acc);
#pragma unroll
        for (int i = 0; i < 4; ++i) y[mt][nt][i] = __builtin_fmaf(sc, acc[i], __builtin_fmaf(off, xs[mt][i], y[mt][nt][i]));
      }
    }
    load(4 * min(i + kRing, ng - 1) + wave, sl);
  };
  for (int ib = 0; ib < ng; ib += kRing) {
#pragma unroll
    for (int j = 0; j < kRing; ++j) step(ib + j, R[j]);
  }

  // the four waves' partial sums (fixed order: wave 0 + 1 + 2 + 3), rounded to bf16 once
  __syncthreads();  // every wave is done with the scale and bias pairs
  if (wave > 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) sm.red[wave - 1][mt * NT + nt][lane] = y[mt][nt];
  }
  __syncthreads();
  if (wave == 0) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        f4 t = y[mt][nt];
#pragma unroll
        for (int w = 0; w < 3; ++w) t = t + sm.red[w][mt * NT + nt][lane];
        if (valid[nt]) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int m = (mt0 + mt) * 16 + 4 * g4 + i;
            if (m < p.M) yr[nt][(size_t)m * ystride[nt]] = f2bf(t[i]);
          }
        }
      }
  }
}

// MFMA path for calls of many weight rows and few operand rows (one m group of up to 48 rows;
// 8 layers or more of in_proj per call): workgroup = 256 weight rows, wave w owns 64 of them
// (kNsTiles 16-row tiles) over the whole of K, and the four waves share the operand, which
// passes through an LDS ring once per workgroup (qgemm_kernel reads it from L2 once per 64
// rows). A step is two groups. Direct-to-LDS loads (`global_load_lds_dwordx4`: lane l's 16
// bytes land at the destination + 16 l, no VGPRs) fill the ring kNsAhead steps ahead: each
// wave issues one of the step's four 1 KB blocks of every m tile, waits for its own loads,
// and one barrier per step then makes the slot whole for all four. Each wave also loads the
// scale words of its rows, 8 groups at a time, into its own pair of LDS buffers (read by that
// wave only: no barrier). The weight words stay in a register ring, loaded and moved into
// fragment order as in qgemm_kernel. Loads complete in issue order and the waits count them,
// so every step issues the same loads (past the last step they repeat it), and no lane is
// masked off in the loop (a divergent branch there split the loop into blocks, after which
// the compiler sank a step's FMAs to its end with every MFMA result live). Per group
// y += s * sum x (128 + q) as in qgemm_kernel, each wave adding its groups in order; the
// bias term sum_g (b_g - 128 s_g) sum x_g is made after the loop as MFMA products (below),
// and each row is rounded once.
constexpr int kNsTiles = 4;
constexpr int kNsRows = 4 * 16 * kNsTiles;  // weight rows per workgroup
constexpr int kNsAhead = 2;                 // steps between a load and its use
typedef __attribute__((address_space(3))) void lds_void;
// Direct-to-LDS loads written as asm: the compiler, which cannot tell which LDS bytes such a
// load writes, otherwise waits for every one in flight (vmcnt(0)) at points in the loop, which
// would undo the ring. The asm statements have a memory clobber (no memory access moves
// across them); the kernel waits for them itself. M0 carries the LDS destination and is
// restored after the load has been issued (the load takes it at issue), so the compiler's
// view of M0 is never disturbed.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p);
}
__device__ __forceinline__ void dma16(const void* src, uint32_t lds) {
  uint32_t m0_saved;
  asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %1, off\n\ts_nop 0\n\ts_mov_b32 m0, %0"
               : "=&s"(m0_saved)
               : "v"(src), "s"(lds)
               : "memory");
}

template <int MT>
__global__ __launch_bounds__(kThreads) void qgemm_ns_kernel(QParams p) {
  constexpr int NT = kNsTiles, D = kNsAhead, S = D + 1;
  constexpr int kSlot = MT * 4 * 1024;     // a slot: [m tile][group of the step][k step] 1 KB operand blocks
  constexpr int kPerStep = MT + 2 * NT;    // vector-memory instructions per wave and step
  constexpr int kMaxG = 8192 / 64;
  __shared__ __attribute__((aligned(16))) unsigned char ring[S * kSlot];
  __shared__ __attribute__((aligned(16))) uint16_t sbl[4][2][64 * 8];  // scale words: [wave][buffer][row][8 groups]
  __shared__ __attribute__((aligned(16))) float xs_all[kMaxG * 16 * MT];  // the sums x: [group][16 MT]

  int bid = blockIdx.x;
  if (p.remap) bid = (bid & 7) * (int)(gridDim.x >> 3) + (bid >> 3);
  const int layer = bid / p.tiles, tile = bid % p.tiles;
  const int lane = threadIdx.x & 63, g4 = lane >> 4, nn = lane & 15;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int K = p.K, G = K / 64, nch = K / 32, nsteps = G / 2, nblk = G / 8;
  const int rbase = (tile * 4 + wave) * 16 * NT;
  const int bsrc = (4 * nn + g4) * 4;  // as in qgemm_kernel
  g_u32x2* wr[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int lrow = rbase + 16 * nt + (lane >> 2);
    const RowPtrs rl = row_ptrs(p, layer, lrow < p.R ? lrow : p.R - 1);
    wr[nt] = (g_u32x2*)(rl.w) + (lane & 3);
  }
  // lane l loads the scale words of the wave's row l
  const RowPtrs rsb = row_ptrs(p, layer, min(rbase + lane, p.R - 1));
  const char* s_src = reinterpret_cast<const char*>(rsb.s);
  const char* xa = reinterpret_cast<const char*>(p.xfrag + (size_t)layer * MT * nch * 512) + 16 * lane;
  // the layer's sums x, all groups, for the bias products after the loop (one barrier: the
  // loop issues no load before it)
  {
    const f4* src = reinterpret_cast<const f4*>(p.xsum + (size_t)layer * G * 16 * MT);
    for (int q = threadIdx.x; q < G * 4 * MT; q += kThreads) reinterpret_cast<f4*>(xs_all)[q] = src[q];
  }
  __syncthreads();
  const NibbleConsts nk = nibble_consts();

  // step j's loads: the wave's block (group 2 j + wave / 2, k step wave % 2) of every m tile
  // and its share of the sums into ring slot sl; its weight words into ws
  const uint32_t ring_l = lds_addr(ring);
  auto issue_op = [&](int j, int sl) {
    const uint32_t dst = ring_l + sl * kSlot;
#pragma unroll
    for (int i = 0; i < MT; ++i) dma16(xa + ((size_t)i * nch + 4 * j + wave) * 1024, dst + (4 * i + wave) * 1024);
  };
  struct WStep {
    u32x2 w[2][NT];
  };
  auto issue_w = [&](int j, WStep& ws) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      g_u32x2* wj = wr[nt] + 8 * j;
      ws.w[0][nt] = wj[0];
      ws.w[1][nt] = wj[4];
    }
  };
  // scale and bias words of groups 8 blk .. + 7 into buffer buf
  const uint32_t sbl_l = lds_addr(&sbl[wave][0][0]);
  auto issue_sb = [&](int blk, int buf) { dma16(s_src + 16 * blk, sbl_l + buf * 1024); };

  f4 y[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) y[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};

  auto compute = [&](int j, const unsigned char* slot, const uint16_t* sbw, const WStep& ws) {
    // the scale words of the step's two groups, one 4-byte read per tile
    uint32_t sw[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) sw[nt] = *reinterpret_cast<const uint32_t*>(sbw + (16 * nt + nn) * 8 + ((2 * j) & 7));
#pragma unroll
    for (int gg = 0; gg < 2; ++gg) {
      bf8 a[MT][2];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int s = 0; s < 2; ++s) a[mt][s] = *reinterpret_cast<const bf8*>(slot + (4 * mt + 2 * gg + s) * 1024 + 16 * lane);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const float sc = __builtin_bit_cast(float, gg ? sw[nt] & 0xFFFF0000u : sw[nt] << 16);
        const uint32_t w0 = (uint32_t)__builtin_amdgcn_ds_bpermute(bsrc, (int)ws.w[gg][nt][0]);
        const uint32_t w1 = (uint32_t)__builtin_amdgcn_ds_bpermute(bsrc, (int)ws.w[gg][nt][1]);
        const bf8 b0 = nibbles_bf16(w0, nk), b1 = nibbles_bf16(w1, nk);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          f4 acc = mfma(a[mt][0], b0, f4{0.f, 0.f, 0.f, 0.f});
          acc = mfma(a[mt][1], b1, acc);
#pragma unroll
          for (int i = 0; i < 4; ++i) y[mt][nt][i] = __builtin_fmaf(sc, acc[i], y[mt][nt][i]);
        }
      }
    }
  };

  WStep W[2];
  issue_sb(0, 0);
#pragma unroll
  for (int j = 0; j < D; ++j) {
    issue_op(j, j);
    issue_w(j, W[j]);
  }
  int sl = 0;  // ring slot of step j
  for (int j0 = 0; j0 < nsteps; j0 += 4) {  // nsteps is a multiple of 4 (G of 8)
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = j0 + r;
      // step j's loads are done once no more than the loads issued after them are in flight:
      // step j + 1's, and also the scale words issued at step 4 b after step 4 b + 2's (in
      // flight at steps 4 b + 1 and 4 b + 2); then every wave's are (the barrier). The wait
      // and the barrier are one asm statement with a memory clobber, so no load moves across
      // them.
      if (r == 1 || r == 2)
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kPerStep + 1) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kPerStep) : "memory");
      compute(j, ring + sl * kSlot, &sbl[wave][(j >> 2) & 1][0], W[r & 1]);
      __builtin_amdgcn_sched_barrier(0);
      // refill what step j - 1 read (every wave is past it: the barrier above)
      const int jn = min(j + D, nsteps - 1);
      issue_op(jn, sl == 0 ? S - 1 : sl - 1);
      issue_w(jn, W[r & 1]);
      if (r == 0) issue_sb(min((j >> 2) + 1, nblk - 1), ((j >> 2) + 1) & 1);
      sl = sl == S - 1 ? 0 : sl + 1;
    }
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the repeated loads, before the LDS goes away
  // this lane's output rows, their scale and bias words: found here rather than held in
  // registers through the loop
  uint16_t* yr[NT];
  const uint16_t *srow[NT], *brow[NT];
  int ystride[NT];
  bool valid[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int grow = rbase + 16 * nt + nn;
    valid[nt] = grow < p.R;
    const RowPtrs rp = row_ptrs(p, layer, valid[nt] ? grow : p.R - 1);
    yr[nt] = rp.y;
    ystride[nt] = rp.ystride;
    srow[nt] = rp.s;
    brow[nt] = rp.b;
  }

  // The bias term sum_g (b_g - 128 s_g) sum x_g = Yb - 128 Ys, Yb = sum_g b_g sum x_g and
  // Ys = sum_g s_g sum x_g, on MFMA after the loop (it was two FMAs per element and group):
  // A = the sums x of 16 operand rows x 32 groups, each split into three bf16 terms (exact to
  // about 2^-24 of it), B = the rows' bias / scale words of the same groups (bf16, exact);
  // groups past G are zeros. Lane (g4, r) takes groups 32 ks + 8 g4 .. + 7.
  {
    f4 yb[MT][NT], ysc[MT][NT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) yb[mt][nt] = ysc[mt][nt] = f4{0.f, 0.f, 0.f, 0.f};
    for (int ks = 0; ks < (G + 31) / 32; ++ks) {
      const int g0 = 32 * ks + 8 * g4;
      const bool live = g0 < G;  // G is a multiple of 16: all eight or none
      bf8 bb[NT], bs[NT];
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        u32x4 vb{}, vs{};
        if (live) {
          const u32x2 b0 = *(g_u32x2*)(brow[nt] + g0), b1 = *(g_u32x2*)(brow[nt] + g0 + 4);
          const u32x2 s0 = *(g_u32x2*)(srow[nt] + g0), s1 = *(g_u32x2*)(srow[nt] + g0 + 4);
          vb = u32x4{b0[0], b0[1], b1[0], b1[1]};
          vs = u32x4{s0[0], s0[1], s1[0], s1[1]};
        }
        bb[nt] = __builtin_bit_cast(bf8, vb);
        bs[nt] = __builtin_bit_cast(bf8, vs);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        float v[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = live ? xs_all[(g0 + i) * 16 * MT + 16 * mt + nn] : 0.0f;
        bf8 hi, mid, lo;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float h = rbf(v[i]);
          const float r1 = v[i] - h;
          const float m1 = rbf(r1);
          hi[i] = __builtin_bit_cast(__bf16, (uint16_t)(__builtin_bit_cast(uint32_t, h) >> 16));
          mid[i] = __builtin_bit_cast(__bf16, (uint16_t)(__builtin_bit_cast(uint32_t, m1) >> 16));
          lo[i] = (__bf16)(r1 - m1);
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          yb[mt][nt] = mfma(hi, bb[nt], yb[mt][nt]);
          yb[mt][nt] = mfma(mid, bb[nt], yb[mt][nt]);
          yb[mt][nt] = mfma(lo, bb[nt], yb[mt][nt]);
          ysc[mt][nt] = mfma(hi, bs[nt], ysc[mt][nt]);
          ysc[mt][nt] = mfma(mid, bs[nt], ysc[mt][nt]);
          ysc[mt][nt] = mfma(lo, bs[nt], ysc[mt][nt]);
        }
      }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int i = 0; i < 4; ++i) y[mt][nt][i] += __builtin_fmaf(-128.0f, ysc[mt][nt][i], yb[mt][nt][i]);
  }

#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      if (valid[nt]) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int m = mt * 16 + 4 * g4 + i;
          if (m < p.M) yr[nt][(size_t)m * ystride[nt]] = f2bf(y[mt][nt][i]);
        }
      }
    }
}

template <bool NORM>
hipError_t launch_j(int J, const QParams& p, dim3 grid, size_t smem, hipStream_t stream) {
  switch (J) {
#define GDN_QL_CASE(j) \
  case j:              \
    hipLaunchKernelGGL((qlinear_kernel<j, NORM>), grid, dim3(kThreads), smem, stream, p); break;
    GDN_QL_CASE(2) GDN_QL_CASE(4) GDN_QL_CASE(8) GDN_QL_CASE(10) GDN_QL_CASE(12) GDN_QL_CASE(16)
#undef GDN_QL_CASE
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

bool qlinear_k_supported(int k) {
  return k == 1024 || k == 2048 || k == 4096 || k == 5120 || k == 6144 || k == 8192;
}

bool qlinear_uses_gemv(int m, int k) {
  return m <= GDN_QLINEAR_GEMV_ROWS && (size_t)m * (k / 32) * (4 * 16 + 4) <= 65536;
}

namespace {
// MFMA path: m-tiles of 16 rows per workgroup (1..4), the m-tile count rounded up to a
// multiple of it (the padding rows are zeros in the workspace)
int qgemm_mt(int m) { return std::min(4, (m + 15) / 16); }
int qgemm_mtiles(int m) {
  const int mt = qgemm_mt(m);
  return ((m + 15) / 16 + mt - 1) / mt * mt;
}

template <int MT>
hipError_t launch_gemm_mt(int NT, const QParams& p, dim3 grid, hipStream_t stream) {
  switch (NT) {
    case 1: hipLaunchKernelGGL((qgemm_kernel<MT, 1>), grid, dim3(kThreads), 0, stream, p); break;
    case 2: hipLaunchKernelGGL((qgemm_kernel<MT, 2>), grid, dim3(kThreads), 0, stream, p); break;
    default: hipLaunchKernelGGL((qgemm_kernel<MT, 4>), grid, dim3(kThreads), 0, stream, p); break;
  }
  return hipGetLastError();
}
}  // namespace

// The no-allocation entry point's workspace: one array per device, held until the process
// ends. Host code never passes `scratch` itself to a kernel (on the host it names a
// stand-in, not device memory): its device address comes from hipGetSymbolAddress, once per
// device with that device current, and only that address is used.
static __device__ __align__(256) unsigned char scratch[GDN_QLINEAR_NOALLOC_SCRATCH_BYTES];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mutex[kMaxScratchDevices];
void* g_scratch_ptr[kMaxScratchDevices];
}  // namespace

// Only a successful lookup is kept: a failure (e.g. before the device's context is usable)
// is returned to this call, and the next call on that device looks the symbol up again.
hipError_t qlinear_scratch(void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mutex[dev]);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (!p) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return hipSuccess;
}

// the operand in fragment order (1 KB per 16 rows x 32 values), then its group sums (fp32
// per row and 64 values)
size_t qlinear_xfrag_bytes(int n_layers, int m, int k) {
  const size_t b = (size_t)n_layers * qgemm_mtiles(m) * (k / 32) * 1024;
  return (b + 255) / 256 * 256;
}
size_t qlinear_workspace_bytes(int n_layers, int m, int k) {
  if (qlinear_uses_gemv(m, k)) return 0;
  const size_t xs = (size_t)n_layers * 16 * qgemm_mtiles(m) * (k / 64) * 4;
  return qlinear_xfrag_bytes(n_layers, m, k) + (xs + 255) / 256 * 256;
}

hipError_t launch_qlinear(const gdn_qlinear_args& a, hipStream_t stream) {
  QParams p{};
  p.M = a.m;
  p.K = a.k;
  p.nseg = a.n_segs;
  p.x = static_cast<const uint16_t*>(a.x);
  p.xf = a.norm_x;
  p.z = static_cast<const uint16_t*>(a.norm_z);
  p.gamma = a.norm_gamma;
  p.eps = a.norm_eps;
  int R = 0;
  for (int q = 0; q < GDN_QLINEAR_MAX_SEGS; ++q) {
    const int qq = q < a.n_segs ? q : 0;  // unused slots repeat segment 0 (never selected)
    p.w[q] = static_cast<const uint32_t*>(a.segs[qq].w);
    p.s[q] = static_cast<const uint16_t*>(a.segs[qq].scales);
    p.b[q] = static_cast<const uint16_t*>(a.segs[qq].biases);
    p.y[q] = static_cast<uint16_t*>(a.segs[qq].y);
    p.n[q] = a.segs[qq].n;
    p.row0[q] = R;
    if (q < a.n_segs) R += a.segs[q].n;
  }
  p.R = R;
  const bool norm = a.norm_x != nullptr;
  if (qlinear_uses_gemv(a.m, a.k)) {
    // rows per workgroup: 64, or 256 with the norm prologue (every workgroup normalises
    // the whole operand, so fewer, taller tiles)
    p.passes = norm ? 16 : 4;
    p.tiles = (R + kRowsPerPass * p.passes - 1) / (kRowsPerPass * p.passes);
    const dim3 grid((unsigned)((size_t)a.n_layers * p.tiles));
    const size_t smem = (size_t)p.M * (a.k / 32) * (4 * 16 + 4);
    return norm ? launch_j<true>(a.k / 512, p, grid, smem, stream) : launch_j<false>(a.k / 512, p, grid, smem, stream);
  }
  // MFMA path: the operand into the workspace, then the product
  const int MT = qgemm_mt(a.m);
  p.mtiles = qgemm_mtiles(a.m);
  p.xfrag = static_cast<uint16_t*>(a.workspace);
  p.xsum = reinterpret_cast<float*>(static_cast<char*>(a.workspace) + qlinear_xfrag_bytes(a.n_layers, a.m, a.k));
  const size_t prep_threads = (size_t)a.n_layers * 16 * p.mtiles * (a.k / 32) * 4;
  const dim3 gp((unsigned)((prep_threads + kThreads - 1) / kThreads));
  if (norm) hipLaunchKernelGGL(qprep_kernel<true>, gp, dim3(kThreads), 0, stream, p, a.n_layers);
  else hipLaunchKernelGGL(qprep_kernel<false>, gp, dim3(kThreads), 0, stream, p, a.n_layers);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int gy = p.mtiles / MT;
  // one m group and enough 256-row workgroups for two per CU: the operand-sharing kernel
  // (its scale and bias loads take 16 bytes a lane)
  bool sb16 = true;
  for (int q = 0; q < a.n_segs; ++q)
    sb16 = sb16 && reinterpret_cast<uintptr_t>(a.segs[q].scales) % 16 == 0 &&
           reinterpret_cast<uintptr_t>(a.segs[q].biases) % 16 == 0;
  const int ns_tiles = (R + kNsRows - 1) / kNsRows;
  if (gy == 1 && MT <= 3 && sb16 && (size_t)a.n_layers * ns_tiles >= 512) {
    p.tiles = ns_tiles;
    p.mgroups = 1;
    const size_t nwg = (size_t)a.n_layers * ns_tiles;
    p.remap = a.n_layers >= 8 && nwg % 8 == 0;
    const dim3 grid((unsigned)nwg);
    switch (MT) {
      case 1: hipLaunchKernelGGL(qgemm_ns_kernel<1>, grid, dim3(kThreads), 0, stream, p); break;
      case 2: hipLaunchKernelGGL(qgemm_ns_kernel<2>, grid, dim3(kThreads), 0, stream, p); break;
      default: hipLaunchKernelGGL(qgemm_ns_kernel<3>, grid, dim3(kThreads), 0, stream, p); break;
    }
    return hipGetLastError();
  }
  // weight rows per workgroup: 64, 32 or 16 -- the most that still gives 512 workgroups
  int NT = 4;
  while (NT > 1 && (size_t)a.n_layers * ((R + 16 * NT - 1) / (16 * NT)) * gy < 512) NT /= 2;
  p.tiles = (R + 16 * NT - 1) / (16 * NT);
  p.mgroups = gy;
  const size_t nwg = (size_t)a.n_layers * p.tiles * gy;
  p.remap = (gy > 1 || a.n_layers >= 8) && nwg % 8 == 0;
  const dim3 grid((unsigned)nwg);
  switch (MT) {
    case 1: return launch_gemm_mt<1>(NT, p, grid, stream);
    case 2: return launch_gemm_mt<2>(NT, p, grid, stream);
    case 3: return launch_gemm_mt<3>(NT, p, grid, stream);
    default: return launch_gemm_mt<4>(NT, p, grid, stream);
  }
}

}  // namespace gdn
