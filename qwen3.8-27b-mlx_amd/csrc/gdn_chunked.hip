// Chunked (WY / UT-transform) prefill of the gated-delta recurrence for gfx950, chunk 64.
//
// For one v-head and a chunk of positions i = 0..63 (python/qwen35.py:365-431):
//   G_i   = sum_{m<=i} log clip(alpha_m, 1e-6, 1)        (within-chunk log decay)
//   A_ij  = beta_i exp(G_i - G_j) (K K^T)_ij, j < i      T' = (I + A)^-1 diag(beta)
//   M_ij  = exp(G_i - G_j) (Q K^T)_ij, j <= i
//   U     = T' V        W = T' diag(e^G) K               (depend on the chunk only)
// and, with the state S as (Dk x Dv) (the transpose of the stored (Dv, Dk) layout):
//   V' = U - W S                                         (= U0 - Kt S of the reference)
//   y  = e^G . (Q S) + M V'                              (= MU0 + Qeff S)
//   S  = e^{G_63} S + K^T (e^{G_63 - G} . V')
//
// Both precisions form V' as
//   V' = T' (V - e^G . (K S))                            (= U - W S)
// so that W and U are never formed; they differ in which products carry their operands
// as bf16 hi + lo (below).
//
// Three kernels, one stream:
//   prefill_frontend  conv + SiLU (+ l2norm, q scale) of every position: q and k into the
//                  fragment planes of Q, K and K^T, and v straight into B-operand fragments
//                  in the interleaved k order (with q, k, v given by the caller,
//                  prefill_vfrag reorders v instead and the intra kernel makes Q, K and
//                  K^T). Extra workgroups of the same launch
//                  compute the gates and each chunk's cumulative log decay G (one wave per
//                  (v-head, chunk)).
//   prefill_intra  one workgroup per (batch, k-head, chunk), all chunks in parallel, three
//                  per CU (two with q, k, v given): K K^T on bf16 MFMA, and for the
//                  k-head's v-heads A, T = (I + A)^-1 (one wave per v-head, fp32, left in
//                  LDS), then each wave's T' fragments from T in LDS, stored as bf16 hi
//                  (and, accurate form, lo) in the register order of the MFMA operands
//                  that read them.
//   prefill_scan   one workgroup per (batch, v-head, pair of 16-column Dv tiles), serial
//                  over the chunks. Each of two state waves keeps its tile's fp32 state
//                  (Dk 128 x Dv 16) in MFMA accumulators and runs the chain (K S,
//                  X = V - e^G K S, V' = T' X), S = e^G63 S + K^T V'' with every operand
//                  in registers; two output waves (position
//                  tiles {0, 3} and {1, 2} of a chunk) run one chunk behind on the S and V'
//                  that the state waves leave in a double-buffered LDS mailbox: one barrier
//                  per chunk. Operands go from the workspace straight into registers two
//                  chunks ahead of their use, and the output waves touch the lines of the
//                  chunk four ahead so that they are in L2 when first asked for. The
//                  output waves build M from the chunk's K and Q. Fast form: K S, Q S,
//                  M V' and K^T V'' use bf16 operands and T' X splits X into bf16 hi + lo
//                  (two MFMAs). Accurate form: S is also split for K S (K is exact in
//                  bf16), T' for T' X (three MFMAs), V'' for K^T V'' (two MFMAs), and M
//                  and V' for M V' (three), so that the state follows the fp32 recurrence
//                  to about 1e-5 instead of 4e-3.
//
// MFMA: v_mfma_f32_16x16x32_bf16. Lane l holds A[l%16][8(l/16)+i], B[8(l/16)+i][l%16]
// and C[4(l/16)+i][l%16] (i < 8, 8, 4). LDS matrices are stored so that both operands
// are read as 16-byte rows ([row][k] for A, [col][k] for B), padded by 8 bf16 per row to
// keep the 16 rows of a fragment on distinct banks. A matrix stored in "fragment order"
// is a sequence of 16 x 32 blocks (row block major, then k block), each block being the
// 64 lanes' 16-byte A fragments in lane order: one 1 KB coalesced load per fragment.
//
// Interleaved k order. The scan's B operands are accumulator tiles: two C tiles stacked
// along k (rows 0..15 and 16..31 of a 32-row k block) give lane l the rows 4(l/16)+i and
// 16+4(l/16)+i, i < 4, of column l%16 -- eight values of the B fragment when the k block
// is read in the order k' = 8g + i <-> k = (i < 4 ? 4g + i : 16 + 4g + i - 4), g = l/16.
// The A operands of those products (W, K and Q over dk, K^T, T' and M over positions) are stored
// in fragment order with their k blocks in that same order, so an accumulator tile turns
// into a B fragment with two conversions and no data movement between lanes.
#include <type_traits>

#include "../../include/gdn.h"
#include "gdn_device_math.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kC = 64;             // chunk
constexpr int kPadB = 8;           // bf16 padding per LDS row
constexpr int kDt = 16;            // Dv columns per scan wave
constexpr int kThreads = 256;
constexpr int kGroup = 3;          // v-heads inverted together (one wave each)
constexpr int kGStride = 128;      // floats per (v-head, chunk) in the gate workspace
constexpr int kFrag = 512;         // bf16 elements of one 16 x 32 fragment block
constexpr int kChunkElems = 8192;  // elements of one chunk's 64 x 128 (or 2 x 64 x 64) matrix

__device__ __forceinline__ f4 mfma(bf8 a, bf8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int LD>
__device__ __forceinline__ bf8 frag(const __bf16 (*m)[LD], int row, int k) {
  return *reinterpret_cast<const bf8*>(&m[row][k]);
}

__device__ __forceinline__ bf4 to_bf4(f4 v) { return __builtin_convertvector(v, bf4); }
__device__ __forceinline__ f4 from_bf4(bf4 v) { return __builtin_convertvector(v, f4); }
// Four fp32 values that already hold bf16 values (low 16 bits zero) as bf16: their high
// halves, two per v_perm_b32 -- the conversion instruction would round them again (2.4
// issue slots a pair, against 1). The elements are copied to scalars first: this compiler
// folds __builtin_bit_cast of an element of a vector value into a cast of element 0.
__device__ __forceinline__ bf4 bf4_of_rounded(f4 v) {
  const float v0 = v[0], v1 = v[1], v2 = v[2], v3 = v[3];
  const uint32_t lo = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, v1), __builtin_bit_cast(uint32_t, v0), 0x07060302u);
  const uint32_t hi = __builtin_amdgcn_perm(__builtin_bit_cast(uint32_t, v3), __builtin_bit_cast(uint32_t, v2), 0x07060302u);
  return __builtin_bit_cast(bf4, (u32x2){lo, hi});
}

// Two accumulator tiles (k rows 0..15 and 16..31 of a block) as one B fragment in the
// interleaved k order.
__device__ __forceinline__ bf8 stack_bf8(f4 lo, f4 hi) {
  return __builtin_shufflevector(to_bf4(lo), to_bf4(hi), 0, 1, 2, 3, 4, 5, 6, 7);
}

typedef float f2v __attribute__((ext_vector_type(2)));
typedef __bf16 bf2v __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));

// Eight fp32 values (two f4, as stack_bf8 orders them) split into bf16 hi (round to nearest
// even) and the bf16 of the remainder, so that hi + lo carries the value to about 2^-16.
// Each pair is converted once (one v_cvt_pk_bf16_f32); the two rounded values the remainder
// needs come back out of the packed word with a shift and a mask (converting each value a
// second time on its own, as from_bf4(to_bf4(x)) compiles, doubled the conversions).
__device__ __forceinline__ void split_bf8(f4 a, f4 b, bf8& hi, bf8& lo) {
  u32x4v w;
  f4 ra, rb;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    w[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){a[2 * j], a[2 * j + 1]}, bf2v));
    w[2 + j] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){b[2 * j], b[2 * j + 1]}, bf2v));
    ra[2 * j] = a[2 * j] - __builtin_bit_cast(float, w[j] << 16);
    ra[2 * j + 1] = a[2 * j + 1] - __builtin_bit_cast(float, w[j] & 0xFFFF0000u);
    rb[2 * j] = b[2 * j] - __builtin_bit_cast(float, w[2 + j] << 16);
    rb[2 * j + 1] = b[2 * j + 1] - __builtin_bit_cast(float, w[2 + j] & 0xFFFF0000u);
  }
  hi = __builtin_bit_cast(bf8, w);
  lo = stack_bf8(ra, rb);
}
// The same for four values.
__device__ __forceinline__ void split_bf4(f4 a, bf4& hi, bf4& lo) {
  uint32_t w[2];
  f4 ra;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    w[j] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f2v){a[2 * j], a[2 * j + 1]}, bf2v));
    ra[2 * j] = a[2 * j] - __builtin_bit_cast(float, w[j] << 16);
    ra[2 * j + 1] = a[2 * j + 1] - __builtin_bit_cast(float, w[j] & 0xFFFF0000u);
  }
  hi = __builtin_bit_cast(bf4, w);
  lo = to_bf4(ra);
}

// e^x for x <= 0 from the hardware 2^x (the decay factors inside a chunk).
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// Offset, in a matrix of `kb` 32-column blocks stored in fragment order with the
// interleaved k order, of element (row, col); col % 4 == 0 addresses 4 consecutive
// elements (8 bytes, one half of a lane's fragment).
__device__ __forceinline__ int ilv_off(int row, int col, int kb) {
  const int o = col & 31;
  return ((row >> 4) * kb + (col >> 5)) * kFrag + ((row & 15) + 16 * ((o & 15) >> 2)) * 8 + 4 * (o >> 4) + (col & 3);
}

// The A fragment of rows row.., k block k0.. in the interleaved k order from an LDS matrix
// stored [row][k]: lane group g = l/16 takes columns k0 + 4g .. +3 and k0 + 16 + 4g .. +3.
template <int LD>
__device__ __forceinline__ bf8 frag_ilv(const __bf16 (*m)[LD], int row, int k0, int g) {
  const bf4 lo = *reinterpret_cast<const bf4*>(&m[row][k0 + 4 * g]);
  const bf4 hi = *reinterpret_cast<const bf4*>(&m[row][k0 + 16 + 4 * g]);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

struct PrefillParams {
  int B, T, Hk, Hv, rep, C, nC;
  int gate_raw, o_bf16;
  int qk_frag;  // the conv front end writes Q, K and K^T straight into ws_q, ws_kk, ws_kt
  int tp_lo;    // T' carried as bf16 hi + lo (GDN_PREFILL_ACCURATE), else hi only
  const uint16_t* x;
  const uint16_t* conv_w;
  const uint16_t* conv_in;
  uint16_t* conv_out;
  const __bf16* q;  // qkv front end (bf16)
  const __bf16* k;
  const __bf16* v;
  const uint16_t* a;
  const uint16_t* b;
  const float* A_log;
  const float* dt_bias;
  const float* alpha;
  const float* beta;
  const float* state_in;
  float* state_out;
  void* o;
  // workspace, per chunk
  // (Q, K, K^T and T' in fragment order with the interleaved k order)
  __bf16* ws_q;   // (B, Hk, nC): Q   (64 x 128)
  __bf16* ws_kt;  // (B, Hk, nC): K^T (128 x 64)
  __bf16* ws_kk;  // (B, Hk, nC): K   (64 x 128), as Q
  __bf16* ws_tp;  // (B, Hv, nC): T' = (I + A)^-1 diag(beta) (64 x 64) in 16 x 32 blocks, bf16
                  // hi and lo blocks alternating (lo written with tp_lo only; the two blocks
                  // above the diagonal are left unwritten)
  float* ws_g;    // (B, Hv, nC, kGStride): (e^G, e^(G63-G)) per position (e^G63 = e^G at 63)
  float* ws_gb;   // (B, Hv, nC, kGStride): (G, beta) per position
  __bf16* ws_vf;  // (B, Hv, nC): V (64 x 128) as B operand fragments in the interleaved k order
                  // (two accumulator tiles of the scan's V - e^G K S): block 2 (dv / 16) + pos / 32, lane 16 g + dv % 16 with
                  // g = (pos % 16) / 4, element (pos % 4) + 4 ((pos % 32) / 16); positions
                  // past T are zeros
};

// Causal depthwise conv from 4 rows (model.cpp:385-395), bf16 after every op.
__device__ __forceinline__ float conv4_rows(float x0, float x1, float x2, float x3, const float (&w)[kTaps]) {
  float y = rbf(x0 * w[0]);
  y = rbf(y + rbf(x1 * w[1]));
  y = rbf(y + rbf(x2 * w[2]));
  y = rbf(y + rbf(x3 * w[3]));
  return y;
}

// Padded conv input rows (absolute position `pos`; negative rows come from the conv
// state, rows past the end are zero). Rows without data read a valid row and are zeroed
// after the load, and the row base is a uniform select, so the loads carry no branches
// and a thread's loads are all in flight together.
__device__ __forceinline__ const uint16_t* xp_base(const PrefillParams& p, int b, int pos) {
  const uint16_t* xr = p.x + ((size_t)b * p.T + min(max(pos, 0), p.T - 1)) * p.C;
  const uint16_t* cr = p.conv_in + ((size_t)b * kConvRows + (kConvRows + pos)) * p.C;
  return (pos < 0 && p.conv_in) ? cr : xr;
}
__device__ __forceinline__ bool xp_valid(const PrefillParams& p, int pos) {
  return pos < p.T && (pos >= 0 || p.conv_in != nullptr);
}

__device__ __forceinline__ uint16_t xp_row(const PrefillParams& p, int b, int pos, int c) {
  const uint16_t v = xp_base(p, b, pos)[c];
  return xp_valid(p, pos) ? v : (uint16_t)0;
}

// Four consecutive channels of the same row (8-byte aligned: C and c are multiples of
// 4, x and the conv state 16-byte aligned).
__device__ __forceinline__ u16x4 xp_vec4(const PrefillParams& p, int b, int pos, int c) {
  const u16x4 v = *reinterpret_cast<const u16x4*>(xp_base(p, b, pos) + c);
  return xp_valid(p, pos) ? v : u16x4{};
}

// ============================================================================ intra

// With the conv front end's fragment planes the kernel needs neither Q nor K^T in LDS: the
// smaller layout (53.8 KB) leaves room for three workgroups per CU (with one group of
// v-heads per k-head, in 165 VGPRs).
struct IntraSmemSlim {
  float G[kGroup][kC];
  float beta[kGroup][kC];
  union {
    struct {
      __bf16 k[kC][kD + kPadB];
    } fe;
    float nat[kGroup][kC][kC + 4];
  } u;
};
struct IntraSmem {
  __bf16 kt[kD][kC + kPadB];  // K^T [dk][pos]
  float G[kGroup][kC];
  float beta[kGroup][kC];
  union {
    struct {
      __bf16 q[kC][kD + kPadB];
      __bf16 k[kC][kD + kPadB];
    } fe;
    // per v-head: -A^T ([j][i] = -A_ij) for the inverse, then T = (I + A)^-1 ([i][j]) over it
    float nat[kGroup][kC][kC + 4];
  } u;
};

// ============================================================================ gates

constexpr int kGateHeads = 4;  // v-heads per gate workgroup (one per wave)

// Gate workgroups per call: (batch, chunk, group of kGateHeads v-heads).
__host__ __device__ __forceinline__ int gate_blocks(int B, int nC, int Hv) {
  return B * nC * ((Hv + kGateHeads - 1) / kGateHeads);
}

// Gates (model.cpp:608-612) and the in-chunk cumulative log decay of one (batch, chunk,
// v-head) per wave, lane = position: G_i = sum_{m<=i} log clip(alpha_m, 1e-6, 1)
// (qwen35.py:397-400). Writes (e^G, e^(G63-G)) to ws_g and (G, beta) to ws_gb. Padded
// steps past T get alpha 1, beta 0 (exact no-ops). Run by extra workgroups of the front-end
// (or v reorder) launch, which have no barriers, so a wave past Hv just returns.
__device__ __forceinline__ void gates_block(const PrefillParams& p, int gb) {
  const int hgroups = (p.Hv + kGateHeads - 1) / kGateHeads;
  const int hg = gb % hgroups;
  gb /= hgroups;
  const int c = gb % p.nC;
  const int b = gb / p.nC;
  const int lane = threadIdx.x & 63;
  const int h = hg * kGateHeads + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (h >= p.Hv) return;
  const int t0 = c * kC, n = min(kC, p.T - t0);
  float al = 1.0f, be = 0.0f;
  if (lane < n) {
    const size_t gi = ((size_t)b * p.T + t0 + lane) * p.Hv + h;
    if (p.gate_raw) {
      d_gates(bf2f(p.a[gi]), bf2f(p.b[gi]), p.A_log[h], p.dt_bias[h], al, be);
    } else {
      al = p.alpha[gi];
      be = p.beta[gi];
    }
  }
  const float ac = al < 1e-6f ? 1e-6f : (al > 1.0f ? 1.0f : al);
  float G = ac == 1.0f ? 0.0f : d_logf(ac);
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const float up = __shfl_up(G, off, 64);
    if (lane >= off) G = G + up;
  }
  const float Gl = __shfl(G, 63, 64);
  const size_t hc = ((size_t)b * p.Hv + h) * p.nC + c;
  reinterpret_cast<float2*>(p.ws_g + hc * kGStride)[lane] = make_float2(d_expf(G), d_expf(Gl - G));
  reinterpret_cast<float2*>(p.ws_gb + hc * kGStride)[lane] = make_float2(G, be);
}

// ============================================================================ front end

constexpr int kFePos = 32;   // positions per front-end workgroup
constexpr int kFeHeads = 4;  // heads of 128 channels per front-end workgroup (one per wave)
static_assert(kC == 2 * kFePos, "a chunk is two front-end position blocks");

// Conv + SiLU, and l2norm for q and k (q also scaled by 128^-0.5), bf16 after every op
// (model.cpp:585-602), into bf16 q (B,T,Hk,128), k (B,T,Hk,128) and v in the fragment order
// of ws_vf.
// Workgroup: (batch, 32 positions, 4 of the 2 Hk + Hv heads in channel order q, k, v);
// wave w takes one head; lane l takes positions 8 (l / 16) .. +7 of the block and the
// head's channels {4m .. 4m+3} and {64+4m .. 64+4m+3}, m = l % 16. The l2norm sum keeps
// the butterfly order of a wave that holds channels (L, L+64) in lane L: lane m adds its
// four pairs as ((p0 + p1) + (p2 + p3)) (the first two butterfly steps), then the DPP
// row sum does the remaining four. The workgroup holding position T-1 also writes the
// conv state hand-off (rows T-3..T-1 of [conv_in ; x]) for its heads.
// A v head's outputs go through the wave's LDS tile ([channel][position]), so that each
// lane then writes eight positions of one channel as one 16-byte piece of the fragment
// order (the q/k and v paths share the conv and SiLU code and their registers). At most 128
// VGPRs: four waves per SIMD for this VALU-bound kernel.
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4))) void prefill_frontend_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) __bf16 vtile[kFeHeads][kD][kFePos + 8];
  const int ngate = gate_blocks(p.B, p.nC, p.Hv);
  if ((int)blockIdx.x < ngate) {  // the gate workgroups come first in the grid
    gates_block(p, blockIdx.x);
    return;
  }
  const int nheads = 2 * p.Hk + p.Hv;
  const int hgroups = (nheads + kFeHeads - 1) / kFeHeads;
  const int pblocks = (p.T + kFePos - 1) / kFePos;
  int bid = blockIdx.x - ngate;
  const int hg = bid % hgroups;
  bid /= hgroups;
  const int pb = bid % pblocks;
  const int b = bid / pblocks;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hh = hg * kFeHeads + wave;
  if (hh >= nheads) return;  // whole waves; the kernel has no barriers
  const int m = lane & 15;
  const int p0 = pb * kFePos + 8 * (lane >> 4);
  const int c0 = hh * kD + 4 * m;
  const int c1 = c0 + 64;
  float w0[4][kTaps], w1[4][kTaps];
#pragma unroll
  for (int j = 0; j < kTaps; ++j) {
    const u16x4 a0 = *reinterpret_cast<const u16x4*>(p.conv_w + (size_t)j * p.C + c0);
    const u16x4 a1 = *reinterpret_cast<const u16x4*>(p.conv_w + (size_t)j * p.C + c1);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w0[e][j] = bf2f(a0[e]);
      w1[e][j] = bf2f(a1[e]);
    }
  }
  u16x4 r0[8 + kConvRows], r1[8 + kConvRows];
#pragma unroll
  for (int i = 0; i < 8 + kConvRows; ++i) {
    r0[i] = xp_vec4(p, b, p0 - kConvRows + i, c0);
    r1[i] = xp_vec4(p, b, p0 - kConvRows + i, c1);
  }
  const bool norm = hh < 2 * p.Hk;
  const bool is_q = hh < p.Hk;
  // Q, K: channels 4 m .. + 3 are group m % 4 of 32-channel block m / 8, in the group's low
  // (m % 8 < 4) or high half
  auto& qt = *reinterpret_cast<__bf16(*)[kFePos][kD + 8]>(&vtile[wave][0][0]);
  const int qcol = 32 * (m >> 3) + 8 * (m & 3) + 4 * ((m >> 2) & 1);
  const bool full_block = (pb + 1) * kFePos <= p.T;  // every position of the block is < T
  const float scale_b = rbf(1.0f / sqrtf((float)kD));
  const float eps_b = rbf(1e-6f);
  auto& vt = vtile[wave];
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    float u[8];  // channels 4m + e (e < 4) and 64 + 4m + (e - 4)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      u[e] = conv4_rows(bf2f(r0[t][e]), bf2f(r0[t + 1][e]), bf2f(r0[t + 2][e]), bf2f(r0[t + 3][e]), w0[e]);
      u[4 + e] = conv4_rows(bf2f(r1[t][e]), bf2f(r1[t + 1][e]), bf2f(r1[t + 2][e]), bf2f(r1[t + 3][e]), w1[e]);
    }
    silu_bf_batch(u);
    const int pos = p0 + t;
    if (norm) {
      f4 y0 = {u[0], u[1], u[2], u[3]}, y1 = {u[4], u[5], u[6], u[7]};
      float pr[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) pr[e] = rbf(u[e] * u[e]) + rbf(u[4 + e] * u[4 + e]);
      const float ssum = rbf(row16_sum((pr[0] + pr[1]) + (pr[2] + pr[3])));
      const float den = rbf(ssum + eps_b);
      const float rs = rsqrt_bf(den);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        y0[e] = rbf(y0[e] * rs);
        y1[e] = rbf(y1[e] * rs);
        if (is_q) {
          y0[e] = rbf(y0[e] * scale_b);
          y1[e] = rbf(y1[e] * scale_b);
        }
      }
      {
        // Q or K to this wave's LDS tile ([position][channel], each 32-channel block in the
        // fragments' interleaved order: channel 32 kb + 4 g + e at 32 kb + 8 g + e and
        // 32 kb + 16 + 4 g + e at 32 kb + 8 g + 4 + e), zeros past T
        const int tp = 8 * (lane >> 4) + t;
        const bool live = pos < p.T;
        *reinterpret_cast<bf4*>(&qt[tp][qcol]) = live ? bf4_of_rounded(y0) : bf4{};
        *reinterpret_cast<bf4*>(&qt[tp][64 + qcol]) = live ? bf4_of_rounded(y1) : bf4{};
      }
    } else {
      // u holds bf16 values: their high halves go to the tile as they are (a 16-bit store of
      // the high half); positions past T are zeros (only the last block has any)
      // (stored as __bf16, the type the tile is read back as)
      const int tp = 8 * (lane >> 4) + t;  // position within the block
      auto hi16 = [](uint32_t b) { return __builtin_bit_cast(__bf16, (uint16_t)(b >> 16)); };
      if (full_block) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vt[4 * m + e][tp] = hi16(__builtin_bit_cast(uint32_t, u[e]));
          vt[64 + 4 * m + e][tp] = hi16(__builtin_bit_cast(uint32_t, u[4 + e]));
        }
      } else {
        const bool live = pos < p.T;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          vt[4 * m + e][tp] = hi16(live ? __builtin_bit_cast(uint32_t, u[e]) : 0u);
          vt[64 + 4 * m + e][tp] = hi16(live ? __builtin_bit_cast(uint32_t, u[4 + e]) : 0u);
        }
      }
    }
  }
  if (!norm) {
    // v into ws_vf (block 2 (dv / 16) + half chunk, lane 16 g + dv % 16: positions 4 g .. +3
    // and 16 + 4 g .. +3 of the half chunk); this wave's LDS tile, written above by this wave
    // only
    const int hv = hh - 2 * p.Hk;
    const int kh = pb & 1;  // which half of the 64-position chunk (kFePos = kC / 2)
    __bf16* vf = p.ws_vf + (((size_t)b * p.Hv + hv) * p.nC + pb / 2) * kChunkElems;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int piece = 64 * i + lane;          // (dv tile, lane of the fragment)
      const int dv = 16 * (piece >> 6) + (lane & 15), pg = lane >> 4;
      const bf4 lo = *reinterpret_cast<const bf4*>(&vt[dv][4 * pg]);
      const bf4 hi = *reinterpret_cast<const bf4*>(&vt[dv][16 + 4 * pg]);
      *reinterpret_cast<bf8*>(vf + (2 * (dv >> 4) + kh) * kFrag + lane * 8) =
          __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      // the last chunk's second half when it lies wholly past T: zeros (no workgroup has
      // positions there, and the scan reads V for every position of a chunk)
      if (kh == 0 && pb == pblocks - 1)
        *reinterpret_cast<bf8*>(vf + (2 * (dv >> 4) + 1) * kFrag + lane * 8) = bf8{};
    }
  }
  if (norm) {
    // Q into ws_q, K into ws_kk: fragment block 4 (position tile) + 32-channel block of the
    // chunk, lane 16 g + r holding position r of the tile, channels 4 g .. + 3 and
    // 16 + 4 g .. + 3 of the block (one 16-byte read of the tile); this block is half a
    // chunk (kFePos = kC / 2)
    const int kh = pb & 1;
    __bf16* qf = (is_q ? p.ws_q : p.ws_kk) + (((size_t)b * p.Hk + (is_q ? hh : hh - p.Hk)) * p.nC + pb / 2) * kChunkElems + lane * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int pt = i >> 2, kb = i & 3;
      *reinterpret_cast<bf8*>(qf + ((2 * kh + pt) * 4 + kb) * kFrag) =
          *reinterpret_cast<const bf8*>(&qt[16 * pt + (lane & 15)][32 * kb + 8 * (lane >> 4)]);
      // the last chunk's second half when it lies wholly past T: zeros
      if (kh == 0 && pb == pblocks - 1) *reinterpret_cast<bf8*>(qf + ((2 + pt) * 4 + kb) * kFrag) = bf8{};
    }
    if (!is_q) {
      // K^T into ws_kt: block 2 (16-channel tile a) + half chunk, lane 16 g + r holding
      // channel 16 a + r at positions 4 g .. + 3 and 16 + 4 g .. + 3 of this block (the B
      // fragment order of V, read down a column of the tile: the channel's column there is
      // 32 (a / 2) + 8 (r / 4) + 4 (a % 2) + r % 4)
      const int r = lane & 15, g = lane >> 4;
      __bf16* ktf = p.ws_kt + (((size_t)b * p.Hk + (hh - p.Hk)) * p.nC + pb / 2) * kChunkElems + lane * 8;
#pragma unroll
      for (int a = 0; a < kD / 16; ++a) {
        const int col = 32 * (a >> 1) + 8 * (r >> 2) + 4 * (a & 1) + (r & 3);
        bf8 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          v[i] = qt[4 * g + i][col];
          v[4 + i] = qt[16 + 4 * g + i][col];
        }
        *reinterpret_cast<bf8*>(ktf + (a * 2 + kh) * kFrag) = v;
        if (kh == 0 && pb == pblocks - 1) *reinterpret_cast<bf8*>(ktf + (a * 2 + 1) * kFrag) = bf8{};
      }
    }
  }
  if (p.conv_out && pb == pblocks - 1) {
    for (int e = lane; e < kConvRows * kD; e += 64) {
      const int r = e / kD, ch = hh * kD + e % kD;
      p.conv_out[((size_t)b * kConvRows + r) * p.C + ch] = xp_row(p, b, p.T - kConvRows + r, ch);
    }
  }
}

// T = (I + A)^-1 of one v-head's strictly lower A (64 x 64), by 16 x 16 blocks, in one
// wave. The buffer holds -A transposed in its upper triangle (nat[j][i] = -A_ij, j < i) and
// receives T in its lower triangle (nat[i][j] = T_ij, i >= j): the two never overlap, so
// -A stays readable while T is written. (1) The four diagonal blocks together, lane = (block
// kb, column c), forward substitution in fp32 (x_r += (-A_rm) x_m for r > m, 120 FMAs a
// lane); their rows are then written whole, zeros above the diagonal. (2) The blocks below,
// a diagonal at a time: T_ij = -T_ii S_ij with S_ij = sum_{k=j}^{i-1} A_ik T_kj, on
// v_mfma_f32_16x16x32_bf16 with both operands split into bf16 hi + lo (three products:
// about 2^-16 relative error). K runs in the interleaved order k' = 8 lg + e <-> row/column
// 4 lg + (e & 3) of the first (e < 4) or second (e >= 4) block of the pair, so the
// accumulator tile S is the B operand of T_ii S as it stands. The blocks above the diagonal
// keep -A^T: the readers of T mask them.
__device__ __forceinline__ void split_bf16(const float (&v)[8], bf8& hi, bf8& lo) {
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const __bf16 h = (__bf16)v[e];
    hi[e] = h;
    lo[e] = (__bf16)(v[e] - (float)h);
  }
}

__device__ __forceinline__ void invert_blocked(float (*nat)[kC + 4], int lane) {
  const int lg = lane >> 4, fr = lane & 15;
  {
    float x[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) x[r] = r == fr ? 1.0f : 0.0f;
#pragma unroll
    for (int m = 0; m < 15; ++m) {
      const float* row = &nat[16 * lg + m][16 * lg];
#pragma unroll
      for (int r4 = (m + 1) & ~3; r4 < 16; r4 += 4) {
        const f4 a = *reinterpret_cast<const f4*>(row + r4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          if (r4 + e > m) x[r4 + e] = __builtin_fmaf(a[e], x[m], x[r4 + e]);
        }
      }
    }
    // (every lane has read its block's -A before any lane writes: one wave, in order)
#pragma unroll
    for (int r = 0; r < 16; ++r) nat[16 * lg + r][16 * lg + fr] = x[r];
  }
  // S += [A_{i,k1} | A_{i,k2}] [T_{k1,j} ; T_{k2,j}] (k2 < 0: one block)
  auto prod = [&](int i, int k1, int k2, int j, f4 acc) -> f4 {
    float av[8], bv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int kk = e < 4 ? k1 : k2;
      const int row = 16 * kk + 4 * lg + (e & 3);
      av[e] = kk < 0 ? 0.0f : -nat[row][16 * i + fr];
      bv[e] = kk < 0 ? 0.0f : nat[row][16 * j + fr];
    }
    bf8 ah, al, bh, bl;
    split_bf16(av, ah, al);
    split_bf16(bv, bh, bl);
    acc = mfma(ah, bh, acc);
    acc = mfma(al, bh, acc);
    acc = mfma(ah, bl, acc);
    return acc;
  };
  // T_ij = -T_ii S, written to the lower triangle
  auto finish = [&](int i, int j, f4 S) {
    const f4 d = *reinterpret_cast<const f4*>(&nat[16 * i + fr][16 * i + 4 * lg]);
    const float av[8] = {d[0], d[1], d[2], d[3], 0.0f, 0.0f, 0.0f, 0.0f};
    const float bv[8] = {S[0], S[1], S[2], S[3], 0.0f, 0.0f, 0.0f, 0.0f};
    bf8 ah, al, bh, bl;
    split_bf16(av, ah, al);
    split_bf16(bv, bh, bl);
    f4 acc = {0.f, 0.f, 0.f, 0.f};
    acc = mfma(ah, bh, acc);
    acc = mfma(al, bh, acc);
    acc = mfma(ah, bl, acc);
#pragma unroll
    for (int t = 0; t < 4; ++t) nat[16 * i + 4 * lg + t][16 * j + fr] = -acc[t];
  };
  const f4 zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < 3; ++j) finish(j + 1, j, prod(j + 1, j, -1, j, zero));
#pragma unroll
  for (int j = 0; j < 2; ++j) finish(j + 2, j, prod(j + 2, j, j + 1, j, zero));
  finish(3, 0, prod(3, 2, -1, 0, prod(3, 0, 1, 0, zero)));
}

// With the conv front end, K comes from the fragment plane it wrote; with q, k, v given they
// are the caller's bf16 (B,T,H,128) rows, and this kernel writes Q, K and K^T in fragment
// order.
// ONE_GROUP: the k-head has at most kGroup v-heads (the K K^T registers are then dead after
// the first group). Everything it writes for the scan is stored non-temporally (on an
// earlier form that wrote 224 MB at T = 4096 this took 62 -> 54 us here and 110 -> 94 us in
// the scan that reads it back). (The front end's outputs, which this kernel reads, stay
// cached: storing them non-temporally made this kernel slower, 54 -> 67 us.)
// FRAGS: the conv front end wrote the fragment planes (p.qk_frag).
template <bool ONE_GROUP, bool FRAGS>
__global__ __launch_bounds__(kThreads, ONE_GROUP && FRAGS ? 3 : 2) void prefill_intra_kernel(PrefillParams p) {
  typedef typename std::conditional<FRAGS, IntraSmemSlim, IntraSmem>::type Smem;
  __shared__ __attribute__((aligned(16))) Smem s;
  const int c = blockIdx.x % p.nC;
  const int rest = blockIdx.x / p.nC;
  const int g = rest % p.Hk;
  const int b = rest / p.Hk;
  const int t0 = c * kC;
  const int n = min(kC, p.T - t0);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, fk = (lane >> 4) * 8, lg = lane >> 4;
  const size_t gc = ((size_t)b * p.Hk + g) * p.nC + c;

  // ---- K (and, from the caller's rows, Q) of the chunk into LDS (bf16); caller rows past
  // the end read the last row and are zeroed, so all the loads are in flight together ----
  {
    constexpr int kIt = kC * kD / 8 / kThreads;
    bf8 qv[kIt], kv[kIt];
    // With the conv front end, K comes from the fragment plane it wrote (zeros past T),
    // thread e taking lane e % 64 of block e / 64; otherwise q, k are the caller's rows.
    if constexpr (!FRAGS) {
#pragma unroll
      for (int it = 0; it < kIt; ++it) {
        const int e = tid + it * kThreads, pos = e / (kD / 8), d8 = (e % (kD / 8)) * 8;
        qv[it] = *reinterpret_cast<const bf8*>(p.q + (((size_t)b * p.T + t0 + min(pos, n - 1)) * p.Hk + g) * kD + d8);
      }
    }
    if constexpr (FRAGS) {
#pragma unroll
      for (int it = 0; it < kIt; ++it)
        kv[it] = *reinterpret_cast<const bf8*>(p.ws_kk + gc * kChunkElems + (size_t)(tid + it * kThreads) * 8);
    } else {
#pragma unroll
      for (int it = 0; it < kIt; ++it) {
        const int e = tid + it * kThreads, pos = e / (kD / 8), d8 = (e % (kD / 8)) * 8;
        kv[it] = *reinterpret_cast<const bf8*>(p.k + (((size_t)b * p.T + t0 + min(pos, n - 1)) * p.Hk + g) * kD + d8);
      }
    }
    // the first group's (G, beta), written by the front end's gate workgroups: wave r takes
    // v-head r, lane = position (loaded behind q and k, so their waits come first)
    const int gs0 = min(kGroup, p.rep);
    float2 gb0 = make_float2(0.0f, 0.0f);
    if (wave < gs0) {
      const size_t hc = ((size_t)b * p.Hv + g * p.rep + wave) * p.nC + c;
      gb0 = reinterpret_cast<const float2*>(p.ws_gb + hc * kGStride)[lane];
    }
    if constexpr (FRAGS) {
      // fragment lane (g, r) of block (position tile pt, 32-channel block kb) of K: position
      // 16 pt + r, channels 32 kb + 4 g .. + 3 and 32 kb + 16 + 4 g .. + 3
#pragma unroll
      for (int it = 0; it < kIt; ++it) {
        const int e = tid + it * kThreads, blk = e >> 6, fl = e & 63;
        const int pos = 16 * (blk >> 2) + (fl & 15), d0 = 32 * (blk & 3) + 4 * (fl >> 4);
        *reinterpret_cast<bf4*>(&s.u.fe.k[pos][d0]) = __builtin_shufflevector(kv[it], kv[it], 0, 1, 2, 3);
        *reinterpret_cast<bf4*>(&s.u.fe.k[pos][d0 + 16]) = __builtin_shufflevector(kv[it], kv[it], 4, 5, 6, 7);
      }
    } else {
#pragma unroll
      for (int it = 0; it < kIt; ++it) {
        const int e = tid + it * kThreads, pos = e / (kD / 8), d8 = (e % (kD / 8)) * 8;
        *reinterpret_cast<bf8*>(&s.u.fe.q[pos][d8]) = pos < n ? qv[it] : bf8{};
      }
#pragma unroll
      for (int it = 0; it < kIt; ++it) {
        const int e = tid + it * kThreads, pos = e / (kD / 8), d8 = (e % (kD / 8)) * 8;
        *reinterpret_cast<bf8*>(&s.u.fe.k[pos][d8]) = pos < n ? kv[it] : bf8{};
      }
    }
    if (wave < gs0) {
      s.G[wave][lane] = gb0.x;
      s.beta[wave][lane] = gb0.y;
    }
  }
  __syncthreads();

  // ---- K K^T on MFMA (wave w: rows j = 16w..; kept in registers); from the caller's rows,
  // also Q and K to the workspace and K^T through LDS to the workspace ----
  f4 gr[4];  // lane: (j = 16 wave + 4 lg + e, i = 16 ct + fr): (K K^T)_ji
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    gr[ct] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks)
      gr[ct] = mfma(frag(s.u.fe.k, 16 * wave + fr, 32 * ks + fk), frag(s.u.fe.k, 16 * ct + fr, 32 * ks + fk), gr[ct]);
  }
  {
    if constexpr (!FRAGS) {
      __bf16* wq = p.ws_q + gc * kChunkElems + lane * 8;
#pragma unroll
      for (int ks = 0; ks < kD / 32; ++ks) {
        __builtin_nontemporal_store(frag_ilv(s.u.fe.q, 16 * wave + fr, 32 * ks, lg),
                                    reinterpret_cast<bf8*>(wq + (wave * 4 + ks) * kFrag));
      }
    }
    if constexpr (!FRAGS) {  // K, in the layout of Q, for the scan's K S
      __bf16* wk = p.ws_kk + gc * kChunkElems + lane * 8;
#pragma unroll
      for (int ks = 0; ks < kD / 32; ++ks) {
        __builtin_nontemporal_store(frag_ilv(s.u.fe.k, 16 * wave + fr, 32 * ks, lg),
                                    reinterpret_cast<bf8*>(wk + (wave * 4 + ks) * kFrag));
      }
    }
    if constexpr (!FRAGS) {  // (else the front end wrote K^T's fragments)
      const int dk = tid & (kD - 1), ph = (tid >> 7) * 32;
#pragma unroll
      for (int q8 = 0; q8 < 4; ++q8) {
        bf8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = s.u.fe.k[ph + 8 * q8 + e][dk];
        *reinterpret_cast<bf8*>(&s.kt[dk][ph + 8 * q8]) = v;
      }
    }
  }
  __syncthreads();
  if constexpr (!FRAGS) {
    __bf16* wkt = p.ws_kt + gc * kChunkElems + lane * 8;
#pragma unroll
    for (int a2 = 0; a2 < 2; ++a2)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int a = 2 * wave + a2;
        __builtin_nontemporal_store(frag_ilv(s.kt, 16 * a + fr, 32 * ks, lg),
                                    reinterpret_cast<bf8*>(wkt + (a * 2 + ks) * kFrag));
      }
  }

  // ---- the k-head's v-heads, in groups of up to three ----
  const int rep_end = ONE_GROUP ? 1 : p.rep;
  for (int r0 = 0; r0 < rep_end; r0 += kGroup) {
    const int gs = min(kGroup, p.rep - r0);
    if (!ONE_GROUP && r0 > 0) {  // a later group's (G, beta) (the first came with q, k)
      if (wave < gs) {
        const size_t hc = ((size_t)b * p.Hv + g * p.rep + r0 + wave) * p.nC + c;
        const float2 gb = reinterpret_cast<const float2*>(p.ws_gb + hc * kGStride)[lane];
        s.G[wave][lane] = gb.x;
        s.beta[wave][lane] = gb.y;
      }
      __syncthreads();
    }

    // A (into LDS as -A^T) from the registers (the scan builds M itself)
    for (int r = 0; r < gs; ++r) {
      const int j0 = 16 * wave + 4 * lg;
      const f4 Gj = *reinterpret_cast<const f4*>(&s.G[r][j0]);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const int i = 16 * ct + fr;
        const float Gi = s.G[r][i], bi = s.beta[r][i];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = j0 + e;
          const float dr = j <= i ? fast_exp(Gi - Gj[e]) : 0.0f;
          s.u.nat[r][j][i] = j < i ? -((bi * dr) * gr[ct][e]) : 0.0f;
        }
      }
    }
    __syncthreads();

    // T = (I + A)^-1: wave r inverts v-head r0 + r in its own slot (T below the diagonal,
    // -A^T left above it)
    if (wave < gs) invert_blocked(s.u.nat[wave], lane);
    __syncthreads();

    for (int r = 0; r < gs; ++r) {
      const int h = g * p.rep + r0 + r;
      const size_t hc = ((size_t)b * p.Hv + h) * p.nC + c;
      // T' = T diag(beta), rows i = 16 wave + fr, as A fragments of the two 32-column
      // blocks kh in the interleaved k order: lane group lg holds the columns
      // j = 32 kh + 4 lg + e and 32 kh + 16 + 4 lg + e (e < 4), the first four in x0, the
      // second in x1. 16-column blocks above row block `wave` still hold -A^T (T is zero
      // there) and are masked; the diagonal blocks were written with zeros above the
      // diagonal.
      auto tprime = [&](int kh, float (&tv)[8]) {
        const float* xr = &s.u.nat[r][16 * wave + fr][32 * kh + 4 * lg];
        const f4 x0 = 2 * kh > wave ? f4{0.f, 0.f, 0.f, 0.f} : *reinterpret_cast<const f4*>(xr);
        const f4 x1 = 2 * kh + 1 > wave ? f4{0.f, 0.f, 0.f, 0.f} : *reinterpret_cast<const f4*>(xr + 16);
        const f4 b0 = *reinterpret_cast<const f4*>(&s.beta[r][32 * kh + 4 * lg]);
        const f4 b1 = *reinterpret_cast<const f4*>(&s.beta[r][32 * kh + 16 + 4 * lg]);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          tv[e] = x0[e] * b0[e];
          tv[4 + e] = x1[e] * b1[e];
        }
      };
      // T' split into bf16 hi + lo (lo stored with tp_lo only), blocks (wave, kh) with
      // kh <= wave / 2 (the others are zero)
      __bf16* wt = p.ws_tp + hc * kChunkElems + lane * 8;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        if (2 * kh > wave) continue;
        float tv[8];
        tprime(kh, tv);
        bf8 th, tl;
        split_bf8(f4{tv[0], tv[1], tv[2], tv[3]}, f4{tv[4], tv[5], tv[6], tv[7]}, th, tl);
        __builtin_nontemporal_store(th, reinterpret_cast<bf8*>(wt + ((wave * 2 + kh) * 2) * kFrag));
        if (p.tp_lo) __builtin_nontemporal_store(tl, reinterpret_cast<bf8*>(wt + ((wave * 2 + kh) * 2 + 1) * kFrag));
      }
    }
    __syncthreads();  // the next group rewrites G, beta and the LDS union
  }
}

// v (B,T,Hv,128) bf16 given by the caller -> ws_vf (the conv front end writes ws_vf itself).
// Workgroup = (batch, v-head, chunk): the 64 x 128 tile goes to LDS transposed ([dv][pos]),
// then each thread writes four 16-byte pieces of eight consecutive positions.
__global__ __launch_bounds__(kThreads) void prefill_vfrag_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) __bf16 vt[kD][kC + kPadB];
  const int ngate = gate_blocks(p.B, p.nC, p.Hv);
  if ((int)blockIdx.x < ngate) {  // whole workgroups: the barrier below is never split
    gates_block(p, blockIdx.x);
    return;
  }
  const int vb = blockIdx.x - ngate;
  const int c = vb % p.nC;
  const int rest = vb / p.nC;
  const int h = rest % p.Hv;
  const int b = rest / p.Hv;
  const int t0 = c * kC, n = min(kC, p.T - t0);
  const int tid = threadIdx.x;
  constexpr int kIt = kC * kD / 8 / kThreads;  // 16-byte pieces per thread
  bf8 raw[kIt];
#pragma unroll
  for (int it = 0; it < kIt; ++it) {
    const int e = tid + it * kThreads, pos = e / (kD / 8), d8 = (e % (kD / 8)) * 8;
    raw[it] = *reinterpret_cast<const bf8*>(p.v + (((size_t)b * p.T + t0 + min(pos, n - 1)) * p.Hv + h) * kD + d8);
  }
#pragma unroll
  for (int it = 0; it < kIt; ++it) {
    const int e = tid + it * kThreads, pos = e / (kD / 8), d8 = (e % (kD / 8)) * 8;
#pragma unroll
    for (int i = 0; i < 8; ++i) vt[d8 + i][pos] = pos < n ? raw[it][i] : (__bf16)0.0f;
  }
  __syncthreads();
  __bf16* vf = p.ws_vf + (((size_t)b * p.Hv + h) * p.nC + c) * kChunkElems;
#pragma unroll
  for (int it = 0; it < kIt; ++it) {
    const int e = tid + it * kThreads;        // (block f, lane l) piece
    const int f = e / 64, l = e % 64;
    const int dv = 16 * (f / 2) + (l & 15), pos = 32 * (f & 1) + 4 * (l >> 4);
    const bf4 lo = *reinterpret_cast<const bf4*>(&vt[dv][pos]);
    const bf4 hi = *reinterpret_cast<const bf4*>(&vt[dv][pos + 16]);
    *reinterpret_cast<bf8*>(vf + e * 8) = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  }
}

// ============================================================================ scan

constexpr int kScanNt = 2;                  // 16-column MFMA tiles per scan workgroup
constexpr int kScanGroups = kD / (kDt * kScanNt);  // scan workgroups per v-head

// What the state wave hands the output waves for one chunk, per lane (lane l's entries are
// written by lane l of the state wave and read by lane l of the output waves): S before
// the chunk as the B operand of Q S, and V'.
template <int NT>
struct ScanMail {
  bf8 sb[NT][kD / 32][64];
  f4 vpr[NT][4][64];
};

// A state wave's share of one chunk's operands, in the register order of the MFMAs that
// read them. The two state waves of a workgroup need all of the chunk's shared operands;
// each loads half and passes it to the other through LDS (ScanShared): K (position tiles
// 2i, 2i + 1), T' (state wave 0 the hi parts of its six nonzero blocks, wave 1 the lo
// parts, which only the accurate form loads) and K^T (dk tiles 4i .. 4i + 3), with the
// wave's own V columns and the gates.
constexpr int kTpBlocks = 6;  // T' blocks (pos tile, pos block): (0,0) (1,0) (2,0) (2,1) (3,0) (3,1)
__device__ __forceinline__ constexpr int tp_tile(int bi) { return bi < 2 ? bi : 2 + (bi - 2) / 2; }
__device__ __forceinline__ constexpr int tp_kb(int bi) { return bi < 2 ? 0 : (bi - 2) % 2; }
struct StateOps {
  bf8 kk[2][4];          // K   [own pos tile][dk block]  (A of K S)
  bf8 tp[kTpBlocks];     // T'  [block], hi (wave 0) or lo (wave 1)  (A of T' X)
  bf8 kt[4][2];          // K^T [own dk tile][pos block]  (A of K^T V'')
  bf8 v[2];              // V   [pos block] of the wave's tile (B order: two accumulator tiles)
  float2 g;              // (e^G, e^(G63-G)) at position `lane`
};

// Output wave `half` makes position tiles half and 3 - half of each chunk: M is lower
// triangular, so the first tile (rows < 32) has one nonzero 32-column block and the second
// two, and both waves get three of the six.
__device__ __forceinline__ constexpr int out_tile(int half, int i) { return i == 0 ? half : 3 - half; }

// An output wave's operands of one chunk: its two position tiles out_tile(half, 0 / 1).
struct OutOps {
  bf8 q[2][4];     // Q [pos tile][dk block]          (A of Q S)
  bf8 m[2][2][2];  // M [pos tile][pos block][hi, lo] (A of M V', built from K and Q; lo in
                   // the accurate form only); [0][1] is zero
  float eg;        // e^G at position `lane`
  float gv;        // G at position `lane`
  unsigned touch[2];  // the cache-line touches issued with this set (see touch_lines)
};

// Chunk operands reach L2 two chunks ahead of their use when the first wave to ask for a
// line finds it already there: every workgroup of a v-head asks for the same lines at the
// same time, so a line fetched on demand costs all of them the full memory latency. The
// output waves therefore touch (one dword per 128-byte line) the lines of the chunk four
// ahead: the v-head's four workgroups split the four 16 KB matrices between them (group
// `grp` takes one: K, T', Q, K^T), and each workgroup touches its own V columns and the gate
// pairs.
__device__ __forceinline__ void touch_lines(const PrefillParams& p, size_t gc, size_t hc, int grp, int jt, int half,
                                            int lane, unsigned (&t)[2]) {
  const unsigned* base;
  if (half == 0) {
    const int r = grp & 3;
    const __bf16* m = r == 0 ? p.ws_kk + gc * kChunkElems
                    : r == 1 ? p.ws_tp + hc * kChunkElems
                    : r == 2 ? p.ws_q + gc * kChunkElems
                             : p.ws_kt + gc * kChunkElems;
    base = reinterpret_cast<const unsigned*>(m);
    t[0] = base[lane * 32];
    t[1] = base[(64 + lane) * 32];
  } else {
    // this workgroup's two dv tiles of V (4 KB, 32 lines) and the (G, beta) pairs
    const unsigned* vb = reinterpret_cast<const unsigned*>(p.ws_vf + hc * kChunkElems + jt * 2 * kFrag);
    const unsigned* gb = reinterpret_cast<const unsigned*>(p.ws_gb + hc * kGStride);
    t[0] = lane < 32 ? vb[lane * 32] : gb[(lane & 3) * 32];
    t[1] = reinterpret_cast<const unsigned*>(p.ws_g + hc * kGStride)[(lane & 3) * 32];
  }
}

// Operand loads for chunk c of the (batch, k-head) gc and (batch, v-head) hc: state wave
// i's halves of K and T' (the accurate form's lo half: wave 1) with its tile's V and the
// gates; its half of K^T follows separately.
template <bool SPLIT>
__device__ __forceinline__ void load_front(const PrefillParams& p, size_t gc, size_t hc, int jt, int i, int lane,
                                           StateOps& op) {
  const __bf16* kk = p.ws_kk + gc * kChunkElems + lane * 8;
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) op.kk[r][ks] = *reinterpret_cast<const bf8*>(kk + ((2 * i + r) * 4 + ks) * kFrag);
  if (SPLIT || i == 0) {
    const __bf16* tp = p.ws_tp + hc * kChunkElems + lane * 8;
#pragma unroll
    for (int bi = 0; bi < kTpBlocks; ++bi)
      op.tp[bi] = *reinterpret_cast<const bf8*>(tp + ((tp_tile(bi) * 2 + tp_kb(bi)) * 2 + i) * kFrag);
  }
  const __bf16* v = p.ws_vf + hc * kChunkElems + lane * 8;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) op.v[kb] = *reinterpret_cast<const bf8*>(v + (2 * jt + kb) * kFrag);
  op.g = reinterpret_cast<const float2*>(p.ws_g + hc * kGStride)[lane];
}
__device__ __forceinline__ void load_qm(const PrefillParams& p, size_t gc, size_t hc, int half, int lane, OutOps& op) {
  const __bf16* q = p.ws_q + gc * kChunkElems + lane * 8;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int pt = out_tile(half, i);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) op.q[i][ks] = *reinterpret_cast<const bf8*>(q + (pt * 4 + ks) * kFrag);
  }
  op.eg = p.ws_g[hc * kGStride + 2 * lane];
  op.gv = p.ws_gb[hc * kGStride + 2 * lane];
}


// The per-position pairs of a wave's gate row `row` (written by this wave) at positions
// 16 pt + 4 (lane / 16) + e, e < 4 (the accumulator-row order): two 16-byte LDS reads, each
// the same address for a lane group (a broadcast) instead of eight lane shuffles.
__device__ __forceinline__ void pair_rows(const float2* row, int pt, int lane, f4& x, f4& y) {
  const f4 a = *reinterpret_cast<const f4*>(row + 16 * pt + 4 * (lane >> 4));
  const f4 b = *reinterpret_cast<const f4*>(row + 16 * pt + 4 * (lane >> 4) + 2);
  x = f4{a[0], a[2], b[0], b[2]};
  y = f4{a[1], a[3], b[1], b[3]};
}

// The operand halves the two state waves exchange, per lane, in two slots: slot c % 2
// holds chunk c's, written during chunk c - 1.
struct ScanShared {
  bf8 kk[3][2][2][4][64];          // [chunk % 3][wave][own pos tile][dk block][lane] (three
                                   // slots: the output waves read chunk c's K during c + 1)
  bf8 kt[2][2][4][2][64];          // [slot][wave][own dk tile][pos block][lane]
  bf8 tp[2][2][kTpBlocks][64];     // [slot][wave (0: hi, 1: lo)][block][lane]
  float2 gt[4][64];                // [wave][position]: the wave's per-position gate pair
};

template <bool SPLIT>
__device__ __forceinline__ void share_out(ScanShared& sh, int slot, int kslot, int i, int lane, const StateOps& nx) {
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) sh.kk[kslot][i][r][ks][lane] = nx.kk[r][ks];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) sh.kt[slot][i][r][ks][lane] = nx.kt[r][ks];
  if (SPLIT || i == 0) {
#pragma unroll
    for (int bi = 0; bi < kTpBlocks; ++bi) sh.tp[slot][i][bi][lane] = nx.tp[bi];
  }
}

// S as the bf16 B fragments of the four dk blocks (and, with `split`, their remainders);
// the bf16 parts also go to the output waves' mail.
template <int NT, bool split>
__device__ __forceinline__ void pack_state(ScanMail<NT>& mb, int i, int lane, const f4 (&S)[kD / 16],
                                           bf8 (&sb)[kD / 32], bf8 (&sbl)[kD / 32]) {
#pragma unroll
  for (int ks = 0; ks < kD / 32; ++ks) {
    if constexpr (split) split_bf8(S[2 * ks], S[2 * ks + 1], sb[ks], sbl[ks]);
    else sb[ks] = stack_bf8(S[2 * ks], S[2 * ks + 1]);
    mb.sb[i][ks][lane] = sb[ks];
  }
}

// The chunk's state update S = e^G63 S + K^T V'' of the wave's tile, V'' = e^(G63 - G) V'
// in bf16 (and, with `split`, its remainder, so that K^T V''_hi + K^T V''_lo carries V''
// at fp32 accuracy: K^T is exact in bf16), with the reloads of the next chunk's operands
// spread between the MFMAs (one load after each: loads issued in a burst queue up in the
// CU's address unit behind the other waves' and hold this wave at the issue). `reload`
// issues the loads of everything but K^T, which follows the last product.
template <int i, bool split, int kLoads, typename Ops, typename Reload>
__device__ __forceinline__ void state_update(const PrefillParams& p, f4 (&S)[kD / 16], const f4 (&vpr)[4],
                                             const f4 (&egr)[4], float gam, const bf8 (&kto)[4][2], Ops& op,
                                             size_t gcn, int lane, Reload reload) {
  bf8 vb[2], vbl[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    const f4 v0 = egr[2 * ks] * vpr[2 * ks], v1 = egr[2 * ks + 1] * vpr[2 * ks + 1];
    if constexpr (split) split_bf8(v0, v1, vb[ks], vbl[ks]);
    else vb[ks] = stack_bf8(v0, v1);
  }
  __builtin_amdgcn_sched_barrier(0);
  reload();
#pragma unroll
  for (int a = 0; a < kD / 16; ++a) S[a] = S[a] * gam;
  // (the eight dk tiles' accumulators interleaved: consecutive MFMAs are independent)
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
    for (int a = 0; a < kD / 16; ++a) {
      const bool own = (a >> 2) == i;
      S[a] = mfma(own ? op.kt[a & 3][ks] : kto[a & 3][ks], vb[ks], S[a]);
    }
    if constexpr (split) {
#pragma unroll
      for (int a = 0; a < kD / 16; ++a) {
        const bool own = (a >> 2) == i;
        S[a] = mfma(own ? op.kt[a & 3][ks] : kto[a & 3][ks], vbl[ks], S[a]);
      }
    }
  }
  {
    const __bf16* kt = p.ws_kt + gcn * kChunkElems + lane * 8;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) op.kt[r][ks] = *reinterpret_cast<const bf8*>(kt + ((4 * i + r) * 2 + ks) * kFrag);
  }
  constexpr int kMfma = split ? 32 : 16;
  constexpr int kPairs = kMfma < kLoads ? kMfma : kLoads;
#pragma unroll
  for (int k = 0; k < kPairs; ++k) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);  // one global load
  }
  if constexpr (kMfma > kPairs) __builtin_amdgcn_sched_group_barrier(0x008, kMfma - kPairs, 0);
  if constexpr (kLoads > kPairs) __builtin_amdgcn_sched_group_barrier(0x020, kLoads - kPairs, 0);
  __builtin_amdgcn_sched_barrier(0);
}

// State wave i of (batch b, v-head h, Dv tile jt): S[a] holds the state's rows dk = 16 a +
// 4 lg + e (lg = lane / 16) of column dv = 16 jt + lane % 16 (S^T as accumulator tiles).
// Chunk c: V' and S = e^G63 S + K^T (e^(G63-G) V'); S before the update and V' go to mail
// slot i. `op` holds this wave's share of chunk c's operands and is reloaded with chunk
// cn's right after their last product; `nx` (chunk c + 1's share, loaded a chunk ago) is
// written to the exchange slot of chunk c + 1.
// V' = T' (V - e^G . (K S)) (with U = T' V and W = T' diag(e^G) K this is U - W S):
// X = V - e^G . K S is formed in fp32 and split into bf16 hi + lo. SPLIT
// (GDN_PREFILL_ACCURATE), at fp32 accuracy: K is exact in bf16 and S is split too
// (K S_hi + K S_lo), and T' X = T'_hi X_hi + T'_lo X_hi + T'_hi X_lo (the dropped T'_lo X_lo
// is 2^-16 relative). Otherwise (GDN_PREFILL_FAST) K S_hi and T'_hi X_hi + T'_hi X_lo.
template <int NT, int i, bool SPLIT>
__device__ __forceinline__ void state_chunk(const PrefillParams& p, ScanMail<NT>& mb, ScanShared& sh,
                                            f4 (&S)[kD / 16], StateOps& op, const StateOps& nx, size_t gcn,
                                            size_t hcn, int jt, int slot, int kslot, int lane) {
  constexpr int o = i ^ 1;
  // the other wave's halves of this chunk's K and K^T, and its part of T' (wave 1 takes
  // wave 0's hi parts; wave 0 takes the lo parts of the accurate form)
  bf8 kko[2][4], kto[4][2], tpo[kTpBlocks];
#pragma unroll
  for (int r = 0; r < 2; ++r)
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) kko[r][ks] = sh.kk[kslot][o][r][ks][lane];
#pragma unroll
  for (int r = 0; r < 4; ++r)
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) kto[r][ks] = sh.kt[slot][o][r][ks][lane];
  if (SPLIT || i == 1) {
#pragma unroll
    for (int bi = 0; bi < kTpBlocks; ++bi) tpo[bi] = sh.tp[slot][o][bi][lane];
  }
  bf8 sb[kD / 32], sbl[kD / 32];
  pack_state<NT, SPLIT>(mb, i, lane, S, sb, sbl);
  sh.gt[i][lane] = op.g;
  f4 eg[4], egr[4];
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) pair_rows(sh.gt[i], pt, lane, eg[pt], egr[pt]);
  const float gam = sh.gt[i][63].x;
  // P = K S_hi (+ K S_lo) for the four position tiles, the accumulators interleaved
  f4 P[4];
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) P[pt] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int ks = 0; ks < kD / 32; ++ks) {
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) {
      const bool own = (pt >> 1) == i;
      P[pt] = mfma(own ? op.kk[pt & 1][ks] : kko[pt & 1][ks], sb[ks], P[pt]);
    }
    if constexpr (SPLIT) {
#pragma unroll
      for (int pt = 0; pt < 4; ++pt) {
        const bool own = (pt >> 1) == i;
        P[pt] = mfma(own ? op.kk[pt & 1][ks] : kko[pt & 1][ks], sbl[ks], P[pt]);
      }
    }
  }
  // X = V - e^G . K S as two B fragments (position blocks) split into bf16 hi + lo
  bf8 xb[2], xbl[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb) {
    const f4 v0 = from_bf4(__builtin_shufflevector(op.v[kb], op.v[kb], 0, 1, 2, 3));
    const f4 v1 = from_bf4(__builtin_shufflevector(op.v[kb], op.v[kb], 4, 5, 6, 7));
    const f4 x0 = v0 - eg[2 * kb] * P[2 * kb], x1 = v1 - eg[2 * kb + 1] * P[2 * kb + 1];
    split_bf8(x0, x1, xb[kb], xbl[kb]);
  }
  // V' = T' X over the six nonzero blocks, three products each (two without T'_lo), in an
  // order that keeps consecutive MFMAs on different accumulators
  f4 vpr[4];
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) vpr[pt] = f4{0.f, 0.f, 0.f, 0.f};
  constexpr int kOrder[kTpBlocks] = {0, 2, 4, 1, 3, 5};
#pragma unroll
  for (int term = 0; term < 3; ++term) {
    if (!SPLIT && term == 1) continue;
#pragma unroll
    for (int j = 0; j < kTpBlocks; ++j) {
      const int bi = kOrder[j], pt = tp_tile(bi), kb = tp_kb(bi);
      const bf8 th = i == 0 ? op.tp[bi] : tpo[bi];
      const bf8 tl = i == 0 ? tpo[bi] : op.tp[bi];
      vpr[pt] = mfma(term == 1 ? tl : th, term == 2 ? xbl[kb] : xb[kb], vpr[pt]);
    }
  }
#pragma unroll
  for (int pt = 0; pt < 4; ++pt) mb.vpr[i][pt][lane] = vpr[pt];
  // 32 (16) MFMAs and 25 loads (K half 8, T' part 6 -- none for the fast form's wave 1 --,
  // V 2, the gates, K^T half 8)
  state_update<i, SPLIT, (SPLIT || i == 0) ? 25 : 19>(p, S, vpr, egr, gam, kto, op, gcn, lane,
                                                      [&] { load_front<SPLIT>(p, gcn, hcn, jt, i, lane, op); });
  share_out<SPLIT>(sh, slot ^ 1, kslot == 2 ? 0 : kslot + 1, i, lane, nx);
  __syncthreads();
}

// Operands are loaded two chunks ahead, in two register sets used by alternate chunks (an
// unrolled pair of chunks per loop trip, so the sets never move between registers), issued
// in the order the loop reissues them so that the loop is entered with the same loads in
// flight as at its back edge. Barriers: one after chunk 0's shares are exchanged, one per
// chunk, one at the end, as the output waves.
template <int NT, int i, bool SPLIT>
__device__ __forceinline__ void scan_state_wave(const PrefillParams& p, ScanMail<NT> (&mail)[2], ScanShared& sh,
                                                int b, int h, int g, int jt, int lane) {
  const int fr = lane & 15, lg = lane >> 4;
  const size_t gc0 = ((size_t)b * p.Hk + g) * p.nC;
  const size_t hc0 = ((size_t)b * p.Hv + h) * p.nC;
  const size_t srow = ((size_t)b * p.Hv + h) * kD * kD + (size_t)(jt * kDt + fr) * kD + 4 * lg;
  // one branch around all the state loads (a branch per load would make the compiler wait
  // for each before the next and for all of them before the operand loads below)
  f4 S[kD / 16];
  if (p.state_in) {
#pragma unroll
    for (int a = 0; a < kD / 16; ++a) S[a] = *reinterpret_cast<const f4*>(p.state_in + srow + 16 * a);
  } else {
#pragma unroll
    for (int a = 0; a < kD / 16; ++a) S[a] = f4{0.f, 0.f, 0.f, 0.f};
  }

  const int last = p.nC - 1;
  StateOps A, B;
  auto load_kt = [&](size_t gc, StateOps& op) {
    const __bf16* kt = p.ws_kt + gc * kChunkElems + lane * 8;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) op.kt[r][ks] = *reinterpret_cast<const bf8*>(kt + ((4 * i + r) * 2 + ks) * kFrag);
  };
  __builtin_amdgcn_sched_barrier(0);
  load_front<SPLIT>(p, gc0, hc0, jt, i, lane, A);
  __builtin_amdgcn_sched_barrier(0);
  load_kt(gc0, A);
  __builtin_amdgcn_sched_barrier(0);
  load_front<SPLIT>(p, gc0 + min(1, last), hc0 + min(1, last), jt, i, lane, B);
  __builtin_amdgcn_sched_barrier(0);
  load_kt(gc0 + min(1, last), B);
  __builtin_amdgcn_sched_barrier(0);
  share_out<SPLIT>(sh, 0, 0, i, lane, A);
  __syncthreads();
  int c = 0, kslot = 0;  // kslot = c % 3 (the accurate form's three K slots)
  for (; c + 2 <= p.nC; c += 2) {
    state_chunk<NT, i, SPLIT>(p, mail[0], sh, S, A, B, gc0 + min(c + 2, last), hc0 + min(c + 2, last), jt, 0, kslot, lane);
    kslot = kslot == 2 ? 0 : kslot + 1;
    state_chunk<NT, i, SPLIT>(p, mail[1], sh, S, B, A, gc0 + min(c + 3, last), hc0 + min(c + 3, last), jt, 1, kslot, lane);
    kslot = kslot == 2 ? 0 : kslot + 1;
  }
  if (c < p.nC) state_chunk<NT, i, SPLIT>(p, mail[0], sh, S, A, B, gc0 + last, hc0 + last, jt, 0, kslot, lane);
  __syncthreads();

  if (p.state_out) {
#pragma unroll
    for (int a = 0; a < kD / 16; ++a) *reinterpret_cast<f4*>(p.state_out + srow + 16 * a) = S[a];
  }
}

// An output wave's staging tile: its 32 positions x NT * 16 columns of the chunk's outputs,
// written in accumulator order and read back as 16-byte pieces of one position's columns.
template <int NT, typename OT>
struct OutTile {
  OT y[32][NT * kDt + 16 / sizeof(OT)];
};

// The outputs of chunk c staged in an output wave's tile to o: lane l stores tile row
// r = l / 2 (position 64 c + 16 out_tile(half, r / 16) + r % 16), columns
// 16 (jt + (l % 2) * NT / 2) ..: NT * 8 consecutive columns, 16 bytes at a time (the tile
// rows were written by this wave).
template <int NT, typename OT>
__device__ __forceinline__ void store_tile(const PrefillParams& p, const OutTile<NT, OT>& tile, int b, int h, int jt,
                                           int half, int c, int lane) {
  constexpr int kPer = NT * kDt / 2;  // columns per lane
  constexpr int kVec = 16 / sizeof(OT);
  const int row = lane >> 1, col = (lane & 1) * kPer;
  const int t = c * kC + 16 * out_tile(half, row >> 4) + (row & 15);
  if (t < p.T) {
    OT* o = static_cast<OT*>(p.o) + ((size_t)b * p.T + t) * p.Hv * kD + (size_t)h * kD + jt * kDt + col;
#pragma unroll
    for (int v = 0; v < kPer / kVec; ++v)
      *reinterpret_cast<f4*>(o + v * kVec) = *reinterpret_cast<const f4*>(&tile.y[row][col + v * kVec]);
  }
}

// Output wave `half` (position tiles out_tile(half, 0 / 1) of each chunk), one chunk behind
// the state wave (chunk c after its barrier c): y = e^G . (Q S) + M V' (with SPLIT, M and V'
// split into bf16 hi + lo) from mail[c % 2] into the tile, after the previous chunk's outputs have been
// stored from it (the stores are issued before the reloads, so a wait for a reloaded
// operand never has to count stores that may not have been issued). `op` is reloaded with
// chunk cn's operands and touches the lines of chunk c + 4 (gc4, hc4). The touches issued
// with this set two chunks ago have long arrived: they are folded into `tacc` only so that
// they stay live.
template <int NT, bool OBF16, bool SPLIT>
__device__ __forceinline__ void output_chunk(const PrefillParams& p, const ScanMail<NT>& mb, ScanShared& sh,
                                             OutTile<NT, typename std::conditional<OBF16, __bf16, float>::type>& tile,
                                             OutOps& op, size_t gcn, size_t hcn, size_t gc4, size_t hc4, int b, int h,
                                             int jt, int half, int c, int kslot, int lane, unsigned& tacc) {
  typedef typename std::conditional<OBF16, __bf16, float>::type OT;
  const int fr = lane & 15, lg = lane >> 4;
  if (c > 0) store_tile<NT, OT>(p, tile, b, h, jt, half, c - 1, lane);
  // Every wave starts its step with LDS reads (the state waves their partner's operand
  // halves, on the chain; these waves K and the mail, ~28 KB each), and the state waves are
  // the critical ones, so these start ~190 cycles later and leave the LDS to the exchange
  // first (accurate form, T = 4096: scan 120 -> 117 us in an A/B run; a longer pause, ~380
  // cycles, gained nothing).
  __builtin_amdgcn_s_sleep(3);
  tacc ^= op.touch[0] ^ op.touch[1];
  // (e^G, G) per position through this wave's gate row
  float2* grow = sh.gt[NT + half];
  grow[lane] = make_float2(op.eg, op.gv);
  f4 eg[2], gr[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) pair_rows(grow, out_tile(half, i), lane, eg[i], gr[i]);
  {
    // M = e^(G_i - G_j) (Q K^T)_ij (j <= i) of this wave's position tiles, from the chunk's K
    // (the state waves' K slot, still unchanged) and Q: tile (j tile, i tile) of K Q^T as an
    // accumulator (rows j), decayed (and, with SPLIT, split into bf16 hi + lo); two stacked j
    // tiles are the A fragment of M's rows i over one 32-position block of j in the
    // interleaved k order.
    // (half is a compile-time constant here: the tiles below the diagonal are known, and
    // their MFMAs, all K fragments read first, interleave)
    constexpr int kJt = 4;
    bf8 kf[kJt][kD / 32];
#pragma unroll
    for (int jt2 = 0; jt2 < kJt; ++jt2)
#pragma unroll
      for (int ks = 0; ks < kD / 32; ++ks)
        if (jt2 <= out_tile(half, 1)) kf[jt2][ks] = sh.kk[kslot][jt2 >> 1][jt2 & 1][ks][lane];
    f4 acc[2][kJt];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int jt2 = 0; jt2 < kJt; ++jt2) acc[i][jt2] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks)
#pragma unroll
      for (int jt2 = 0; jt2 < kJt; ++jt2)
#pragma unroll
        for (int i = 0; i < 2; ++i)
          if (jt2 <= out_tile(half, i)) acc[i][jt2] = mfma(kf[jt2][ks], op.q[i][ks], acc[i][jt2]);
    f4 gj[kJt];
#pragma unroll
    for (int jt2 = 0; jt2 < kJt; ++jt2) {
      if (jt2 == out_tile(half, 0)) gj[jt2] = gr[0];
      else if (jt2 == out_tile(half, 1)) gj[jt2] = gr[1];
      else {
        f4 unused;
        pair_rows(grow, jt2, lane, unused, gj[jt2]);
      }
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int pt = out_tile(half, i);
      const float gi = grow[16 * pt + fr].y;
#pragma unroll
      for (int kb = 0; kb <= i; ++kb) {
        f4 mt[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
          const int jt2 = 2 * kb + hh;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int j = 16 * jt2 + 4 * lg + e;
            mt[hh][e] = jt2 <= pt && j <= 16 * pt + fr ? fast_exp(gi - gj[jt2][e]) * acc[i][jt2][e] : 0.0f;
          }
        }
        if constexpr (SPLIT) split_bf8(mt[0], mt[1], op.m[i][kb][0], op.m[i][kb][1]);
        else op.m[i][kb][0] = stack_bf8(mt[0], mt[1]);
      }
    }
  }
#pragma unroll
  for (int n = 0; n < NT; ++n) {
    bf8 sb[kD / 32];
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks) sb[ks] = mb.sb[n][ks][lane];
    f4 vpr[4];
#pragma unroll
    for (int pt = 0; pt < 4; ++pt) vpr[pt] = mb.vpr[n][pt][lane];
    bf8 vh[2], vl[2];
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      if constexpr (SPLIT) split_bf8(vpr[2 * ks], vpr[2 * ks + 1], vh[ks], vl[ks]);
      else vh[ks] = stack_bf8(vpr[2 * ks], vpr[2 * ks + 1]);
    }
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      f4 qs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kD / 32; ++ks) qs = mfma(op.q[i][ks], sb[ks], qs);
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks <= i; ++ks) {  // (M's block (tile 0 or 1, columns 32..63) is zero)
        acc = mfma(op.m[i][ks][0], vh[ks], acc);
        if constexpr (SPLIT) {
          acc = mfma(op.m[i][ks][1], vh[ks], acc);
          acc = mfma(op.m[i][ks][0], vl[ks], acc);
        }
      }
      const f4 y = eg[i] * qs + acc;
#pragma unroll
      for (int e = 0; e < 4; ++e) tile.y[16 * i + 4 * lg + e][16 * n + fr] = (OT)y[e];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  load_qm(p, gcn, hcn, half, lane, op);
  touch_lines(p, gc4, hc4, jt / NT, jt, half, lane, op.touch);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();  // done with mail[c % 2]; mail[(c + 1) % 2] is complete
}

template <int NT, bool OBF16, bool SPLIT, int HALF>
__device__ __forceinline__ void scan_output_wave(const PrefillParams& p, const ScanMail<NT> (&mail)[2], ScanShared& sh,
                                                 OutTile<NT, typename std::conditional<OBF16, __bf16, float>::type>& tile,
                                                 int b, int h, int g, int jt, int lane) {
  constexpr int half = HALF;
  typedef typename std::conditional<OBF16, __bf16, float>::type OT;
  const size_t gc0 = ((size_t)b * p.Hk + g) * p.nC;
  const size_t hc0 = ((size_t)b * p.Hv + h) * p.nC;
  const int last = p.nC - 1;
  const int grp = jt / NT;
  unsigned tacc = 0;
  OutOps A, B;
  __builtin_amdgcn_sched_barrier(0);
  load_qm(p, gc0, hc0, half, lane, A);
  touch_lines(p, gc0 + min(2, last), hc0 + min(2, last), grp, jt, half, lane, A.touch);
  __builtin_amdgcn_sched_barrier(0);
  load_qm(p, gc0 + min(1, last), hc0 + min(1, last), half, lane, B);
  touch_lines(p, gc0 + min(3, last), hc0 + min(3, last), grp, jt, half, lane, B.touch);
  __builtin_amdgcn_sched_barrier(0);
  __syncthreads();  // the state waves' exchange of chunk 0's shares
  __syncthreads();  // chunk 0's mail
  int c = 0, kslot = 0;  // kslot = c % 3
  for (; c + 2 <= p.nC; c += 2) {
    output_chunk<NT, OBF16, SPLIT>(p, mail[0], sh, tile, A, gc0 + min(c + 2, last), hc0 + min(c + 2, last),
                            gc0 + min(c + 4, last), hc0 + min(c + 4, last), b, h, jt, half, c, kslot, lane, tacc);
    kslot = kslot == 2 ? 0 : kslot + 1;
    output_chunk<NT, OBF16, SPLIT>(p, mail[1], sh, tile, B, gc0 + min(c + 3, last), hc0 + min(c + 3, last),
                            gc0 + min(c + 5, last), hc0 + min(c + 5, last), b, h, jt, half, c + 1, kslot, lane, tacc);
    kslot = kslot == 2 ? 0 : kslot + 1;
  }
  if (c < p.nC)
    output_chunk<NT, OBF16, SPLIT>(p, mail[0], sh, tile, A, gc0 + last, hc0 + last, gc0 + last, hc0 + last, b, h, jt, half,
                            c, kslot, lane, tacc);
  store_tile<NT, OT>(p, tile, b, h, jt, half, p.nC - 1, lane);
  // (never true: T >= 1; it keeps the touches from being dropped as unused)
  if (tacc == 0x9e3779b9u && p.T < 0) static_cast<float*>(p.o)[lane] = 0.0f;
}

// Workgroup = (batch, v-head, NT 16-column Dv tiles): waves 0 .. NT-1 carry the state of
// one tile each, waves NT and NT + 1 make the outputs of position tiles {0, 3} and {1, 2}
// of each chunk for all NT tiles. All waves pass nC + 2 barriers.
// SPLIT: GDN_PREFILL_ACCURATE's hi + lo operands.
template <int NT, bool OBF16, bool SPLIT>
__global__ __launch_bounds__(64 * (NT + 2)) void prefill_scan_kernel(PrefillParams p) {
  typedef typename std::conditional<OBF16, __bf16, float>::type OT;
  static_assert(NT == 2, "two state waves exchange halves of K, K^T and T'");
  __shared__ __attribute__((aligned(16))) ScanMail<NT> mail[2];
  __shared__ __attribute__((aligned(16))) OutTile<NT, OT> tiles[2];
  __shared__ __attribute__((aligned(16))) ScanShared shared_ops;
  // Workgroups are dispatched to the 8 XCDs round robin (bid % 8); renumber them so that
  // each XCD gets a contiguous range of (batch, v-head, tiles) -- whole v-heads, and whole
  // k-head groups when the count divides -- and the chunk operands those waves share are
  // fetched into one L2.
  constexpr int kGroups = kD / (kDt * NT);
  int bid = blockIdx.x;
  if ((gridDim.x & 7) == 0) bid = (bid & 7) * (gridDim.x >> 3) + (bid >> 3);
  const int jt = (bid % kGroups) * NT;
  const int rest = bid / kGroups;
  const int h = rest % p.Hv;
  const int b = rest / p.Hv;
  const int g = h / p.rep;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (wave == 0) {
    scan_state_wave<NT, 0, SPLIT>(p, mail, shared_ops, b, h, g, jt, lane);
  } else if (wave == 1) {
    scan_state_wave<NT, 1, SPLIT>(p, mail, shared_ops, b, h, g, jt + 1, lane);
  } else if (wave == NT) {
    scan_output_wave<NT, OBF16, SPLIT, 0>(p, mail, shared_ops, tiles[0], b, h, g, jt, lane);
  } else {
    scan_output_wave<NT, OBF16, SPLIT, 1>(p, mail, shared_ops, tiles[1], b, h, g, jt, lane);
  }
}

struct WorkspaceLayout {
  size_t q, kt, g, vf, gb, kk, tp, total;
};

// The conv front end writes Q, K and K^T straight into their fragment planes and v into vf
// (the qkv front end fills vf from the caller's v; its Q, K and K^T come from the intra
// kernel). Per chunk also T' (hi + lo; the fast form leaves the lo blocks unused). The
// same layout serves both precisions and both front ends.
WorkspaceLayout workspace_layout(int B, int T, int Hk, int Hv) {
  const size_t nC = (size_t)(T + kC - 1) / kC;
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t qk = al((size_t)B * Hk * nC * kChunkElems * 2);
  const size_t wm = al((size_t)B * Hv * nC * kChunkElems * 2);
  const size_t gg = al((size_t)B * Hv * nC * kGStride * 4);
  WorkspaceLayout L{};
  L.q = 0;
  L.kt = L.q + qk;
  L.g = L.kt + qk;
  L.vf = L.g + gg;
  L.gb = L.vf + wm;
  L.kk = L.gb + gg;
  L.tp = L.kk + qk;
  L.total = L.tp + wm;
  return L;
}

}  // namespace

size_t prefill_workspace_bytes(int B, int T, int Hk, int Hv) {
  return workspace_layout(B, T, Hk, Hv).total;
}

hipError_t launch_chunked_prefill(const gdn_layer_args& a, void* workspace, hipStream_t stream,
                                  hipEvent_t* events) {
  PrefillParams p{};
  p.B = a.batch;
  p.T = a.seq_len;
  p.Hk = a.num_k_heads;
  p.Hv = a.num_v_heads;
  p.rep = p.Hv / p.Hk;
  p.C = 2 * p.Hk * kD + p.Hv * kD;
  p.nC = (p.T + kC - 1) / kC;
  p.gate_raw = a.gate_mode == GDN_GATES_RAW;
  p.qk_frag = a.frontend == GDN_FRONTEND_CONV;
  p.tp_lo = a.prefill_precision == GDN_PREFILL_ACCURATE;
  p.o_bf16 = a.o_dtype == GDN_DTYPE_BF16;
  p.x = static_cast<const uint16_t*>(a.x);
  p.conv_w = static_cast<const uint16_t*>(a.conv_weight);
  p.conv_in = static_cast<const uint16_t*>(a.conv_state_in);
  p.conv_out = static_cast<uint16_t*>(a.conv_state_out);
  p.q = static_cast<const __bf16*>(a.q);
  p.k = static_cast<const __bf16*>(a.k);
  p.v = static_cast<const __bf16*>(a.v);
  p.a = static_cast<const uint16_t*>(a.a);
  p.b = static_cast<const uint16_t*>(a.b);
  p.A_log = a.A_log;
  p.dt_bias = a.dt_bias;
  p.alpha = a.alpha;
  p.beta = a.beta;
  p.state_in = a.state_in;
  p.state_out = a.state_out;
  p.o = a.o;
  const bool conv = a.frontend == GDN_FRONTEND_CONV;
  const WorkspaceLayout L = workspace_layout(p.B, p.T, p.Hk, p.Hv);
  char* w = static_cast<char*>(workspace);
  p.ws_q = reinterpret_cast<__bf16*>(w + L.q);
  p.ws_kt = reinterpret_cast<__bf16*>(w + L.kt);
  p.ws_kk = reinterpret_cast<__bf16*>(w + L.kk);
  p.ws_tp = reinterpret_cast<__bf16*>(w + L.tp);
  p.ws_gb = reinterpret_cast<float*>(w + L.gb);
  p.ws_g = reinterpret_cast<float*>(w + L.g);
  p.ws_vf = reinterpret_cast<__bf16*>(w + L.vf);
  if (conv) {
    // the front end writes Q, K and K^T into ws_q, ws_kk and ws_kt and v into ws_vf
    p.q = p.k = p.v = nullptr;
  }

  const dim3 block(kThreads);
  const size_t ngate = (size_t)gate_blocks(p.B, p.nC, p.Hv);
  const dim3 g1((unsigned)((size_t)p.B * p.Hk * p.nC));
  const dim3 g2((unsigned)((size_t)p.B * p.Hv * kScanGroups));
  // events[0..3] (when given) are recorded before the first kernel and after each
  auto mark = [&](int i) {
    if (events) (void)hipEventRecord(events[i], stream);
  };
  mark(0);
  if (conv) {
    const size_t nh = ((size_t)2 * p.Hk + p.Hv + kFeHeads - 1) / kFeHeads;
    const dim3 g0((unsigned)(ngate + (size_t)p.B * ((p.T + kFePos - 1) / kFePos) * nh));
    hipLaunchKernelGGL(prefill_frontend_kernel, g0, block, 0, stream, p);
  } else {
    const dim3 gv((unsigned)(ngate + (size_t)p.B * p.Hv * p.nC));
    hipLaunchKernelGGL(prefill_vfrag_kernel, gv, block, 0, stream, p);
  }
  mark(1);
  // <one group of v-heads per k-head, the front end's fragment planes>
#define GDN_INTRA(og, fr) hipLaunchKernelGGL((prefill_intra_kernel<og, fr>), g1, block, 0, stream, p)
  const bool one = p.rep <= kGroup, fr = p.qk_frag != 0;
  if (one) { if (fr) GDN_INTRA(true, true); else GDN_INTRA(true, false); }
  else { if (fr) GDN_INTRA(false, true); else GDN_INTRA(false, false); }
#undef GDN_INTRA
  mark(2);
  const dim3 sb(64 * (kScanNt + 2));
  if (p.o_bf16) {
    if (p.tp_lo) hipLaunchKernelGGL((prefill_scan_kernel<kScanNt, true, true>), g2, sb, 0, stream, p);
    else hipLaunchKernelGGL((prefill_scan_kernel<kScanNt, true, false>), g2, sb, 0, stream, p);
  } else {
    if (p.tp_lo) hipLaunchKernelGGL((prefill_scan_kernel<kScanNt, false, true>), g2, sb, 0, stream, p);
    else hipLaunchKernelGGL((prefill_scan_kernel<kScanNt, false, false>), g2, sb, 0, stream, p);
  }
  mark(3);
  return hipGetLastError();
}

}  // namespace gdn
