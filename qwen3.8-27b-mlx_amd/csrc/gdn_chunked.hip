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
// Three kernels, one stream:
//   prefill_frontend  conv + SiLU (+ l2norm, q scale) of every position into bf16 q, k
//                  (B, T, Hk, 128) and v, which goes straight into the fragment order of
//                  U's B operand (with q, k, v given by the caller, prefill_vfrag reorders
//                  v instead).
//   prefill_intra  one workgroup per (batch, k-head, chunk), all chunks in parallel, two
//                  per CU: K K^T and K Q^T on bf16 MFMA, and for the k-head's v-heads the
//                  gates, A and M, T = (I + A)^-1 (one wave per v-head, fp32, left in LDS),
//                  U = T'V and W = T'diag(e^G)K on bf16 MFMA, every wave building its T'
//                  fragments from T in LDS (T' split into bf16 hi + lo for U). Results go
//                  to the workspace, already in the register order of the MFMA operands
//                  that read them.
//   prefill_scan   one workgroup per (batch, v-head, 32-column Dv tile), serial over the
//                  chunks; the fp32 state tile lives in MFMA accumulators. Each chunk's
//                  operands go from the workspace straight into registers, two chunks
//                  ahead of their use; LDS holds only the operands all four waves share
//                  (S^T and V'). W S, Q S and K^T V'' use bf16 operands; M V' splits both
//                  operands into bf16 hi + lo (three MFMAs).
//
// MFMA: v_mfma_f32_16x16x32_bf16. Lane l holds A[l%16][8(l/16)+i], B[8(l/16)+i][l%16]
// and C[4(l/16)+i][l%16] (i < 8, 8, 4). LDS matrices are stored so that both operands
// are read as 16-byte rows ([row][k] for A, [col][k] for B), padded by 8 bf16 per row to
// keep the 16 rows of a fragment on distinct banks. A matrix stored in "fragment order"
// is a sequence of 16 x 32 blocks (row block major, then k block), each block being the
// 64 lanes' 16-byte A fragments in lane order: one 1 KB coalesced load per fragment.
#include "../../include/gdn.h"
#include "gdn_device_math.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint16_t u16x4 __attribute__((ext_vector_type(4)));

constexpr int kC = 64;             // chunk
constexpr int kPadB = 8;           // bf16 padding per LDS row
constexpr int kDt = 32;            // Dv columns per scan workgroup
constexpr int kThreads = 256;
constexpr int kGroup = 3;          // v-heads inverted together (one wave each)
constexpr int kGStride = 132;      // floats per (v-head, chunk) in the gate workspace
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

// e^x for x <= 0 from the hardware 2^x (the decay factors inside a chunk).
__device__ __forceinline__ float fast_exp(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

// Offset, in a matrix of `kb` 32-column blocks stored in fragment order, of element
// (row, col); col % 4 == 0 addresses 4 consecutive elements (8 bytes).
__device__ __forceinline__ int frag_off(int row, int col, int kb) {
  return ((row >> 4) * kb + (col >> 5)) * kFrag + ((row & 15) + 16 * ((col & 31) >> 3)) * 8 + (col & 7);
}

struct PrefillParams {
  int B, T, Hk, Hv, rep, C, nC;
  int gate_raw, o_bf16;
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
  __bf16* ws_q;   // (B, Hk, nC): Q   (64 x 128) in fragment order
  __bf16* ws_kt;  // (B, Hk, nC): K^T (128 x 64) in fragment order
  __bf16* ws_w;   // (B, Hv, nC): W   (64 x 128) in fragment order
  __bf16* ws_m;   // (B, Hv, nC): M   (64 x 64) in fragment order, hi and lo blocks interleaved
  float* ws_u;    // (B, Hv, nC): U   (64 x 128) as MFMA result tiles [dv tile][pos tile][lane][4]
  float* ws_g;    // (B, Hv, nC, kGStride): e^G [64], e^(G63-G) [64], e^G63
  __bf16* ws_vf;  // (B, Hv, nC): V (64 x 128) as the B operand of U = T' V, in fragment order:
                  // block 2 (dv / 16) + pos / 32, lane 16 ((pos % 32) / 8) + dv % 16, element
                  // pos % 8; positions past T are zeros
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

struct IntraSmem {
  __bf16 kt[kD][kC + kPadB];  // K^T [dk][pos]
  float G[kGroup][kC];
  float beta[kGroup][kC];
  float eG[kGroup][kC];  // e^G
  union {
    struct {
      __bf16 q[kC][kD + kPadB];
      __bf16 k[kC][kD + kPadB];
    } fe;
    // per v-head: -A^T ([j][i] = -A_ij) for the inverse, then T = (I + A)^-1 ([i][j]) over it
    float nat[kGroup][kC][kC + 4];
  } u;
};

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
  const int nheads = 2 * p.Hk + p.Hv;
  const int hgroups = (nheads + kFeHeads - 1) / kFeHeads;
  const int pblocks = (p.T + kFePos - 1) / kFePos;
  int bid = blockIdx.x;
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
  __bf16* dst = nullptr;
  if (is_q) dst = const_cast<__bf16*>(p.q) + ((size_t)b * p.T * p.Hk + hh) * kD;
  else if (norm) dst = const_cast<__bf16*>(p.k) + ((size_t)b * p.T * p.Hk + (hh - p.Hk)) * kD;
  const size_t pstride = (size_t)p.Hk * kD;
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
      const float rs = rbf(1.0f / sqrtf(den));
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        y0[e] = rbf(y0[e] * rs);
        y1[e] = rbf(y1[e] * rs);
        if (is_q) {
          y0[e] = rbf(y0[e] * scale_b);
          y1[e] = rbf(y1[e] * scale_b);
        }
      }
      if (pos < p.T) {
        __bf16* o = dst + (size_t)pos * pstride;
        *reinterpret_cast<bf4*>(o + 4 * m) = to_bf4(y0);
        *reinterpret_cast<bf4*>(o + 64 + 4 * m) = to_bf4(y1);
      }
    } else {
      const int tp = 8 * (lane >> 4) + t;  // position within the block
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        vt[4 * m + e][tp] = pos < p.T ? (__bf16)u[e] : (__bf16)0.0f;
        vt[64 + 4 * m + e][tp] = pos < p.T ? (__bf16)u[4 + e] : (__bf16)0.0f;
      }
    }
  }
  if (!norm) {
    // v: the B operand of U = T' V in fragment order (block 2 (dv / 16) + half chunk, lane
    // 16 (position / 8) + dv % 16); this wave's LDS tile, written above by this wave only
    const int hv = hh - 2 * p.Hk;
    const int kh = pb & 1;  // which half of the 64-position chunk (kFePos = kC / 2)
    __bf16* vf = p.ws_vf + (((size_t)b * p.Hv + hv) * p.nC + pb / 2) * kChunkElems;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const int piece = 64 * i + lane;          // (dv tile, lane of the fragment)
      const int dv = 16 * (piece >> 6) + (lane & 15), pg = lane >> 4;
      *reinterpret_cast<bf8*>(vf + (2 * (dv >> 4) + kh) * kFrag + lane * 8) =
          *reinterpret_cast<const bf8*>(&vt[dv][8 * pg]);
    }
  }
  if (p.conv_out && pb == pblocks - 1) {
    for (int e = lane; e < kConvRows * kD; e += 64) {
      const int r = e / kD, ch = hh * kD + e % kD;
      p.conv_out[((size_t)b * kConvRows + r) * p.C + ch] = xp_row(p, b, p.T - kConvRows + r, ch);
    }
  }
}

// Column j (this lane) of T = (I + A)^-1 by forward substitution, right-looking: once x_m
// is final, x_i += (-A_im) x_m for every later row i. All lanes read the same LDS words.
__device__ __forceinline__ void invert_column(const float (*nat)[kC + 4], int j, float (&x)[kC]) {
#pragma unroll
  for (int i = 0; i < kC; ++i) x[i] = i == j ? 1.0f : 0.0f;
#pragma unroll
  for (int m = 0; m < kC - 1; ++m) {
#pragma unroll
    for (int i4 = (m + 1) & ~3; i4 < kC; i4 += 4) {
      const f4 a = *reinterpret_cast<const f4*>(&nat[m][i4]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (i4 + e > m) x[i4 + e] = __builtin_fmaf(a[e], x[m], x[i4 + e]);
      }
    }
  }
}

// q, k, v are bf16 (B,T,H,128) -- the caller's, or the front-end kernel's output.
// ONE_GROUP: the k-head has at most kGroup v-heads (the K K^T / Q K^T registers are then
// dead after the first group).
template <bool ONE_GROUP>
__global__ __launch_bounds__(kThreads, 2) void prefill_intra_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) IntraSmem s;
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

  // ---- q, k of the chunk into LDS (bf16); rows past the end read the last row and are
  // zeroed, so all eight loads are in flight together ----
  {
    constexpr int kIt = kC * kD / 8 / kThreads;
    bf8 qv[kIt], kv[kIt];
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int e = tid + it * kThreads, pos = e / (kD / 8), d8 = (e % (kD / 8)) * 8;
      const size_t gi = (((size_t)b * p.T + t0 + min(pos, n - 1)) * p.Hk + g) * kD + d8;
      qv[it] = *reinterpret_cast<const bf8*>(p.q + gi);
      kv[it] = *reinterpret_cast<const bf8*>(p.k + gi);
    }
#pragma unroll
    for (int it = 0; it < kIt; ++it) {
      const int e = tid + it * kThreads, pos = e / (kD / 8), d8 = (e % (kD / 8)) * 8;
      *reinterpret_cast<bf8*>(&s.u.fe.q[pos][d8]) = pos < n ? qv[it] : bf8{};
      *reinterpret_cast<bf8*>(&s.u.fe.k[pos][d8]) = pos < n ? kv[it] : bf8{};
    }
  }
  __syncthreads();

  // ---- K K^T and K Q^T on MFMA (wave w: rows j = 16w..; kept in registers), Q to the
  // workspace, K^T into LDS ----
  f4 gr[4], kq[4];  // lane: (j = 16 wave + 4 lg + e, i = 16 ct + fr): (K K^T)_ji, (Q K^T)_ij
#pragma unroll
  for (int ct = 0; ct < 4; ++ct) {
    gr[ct] = f4{0.f, 0.f, 0.f, 0.f};
    kq[ct] = gr[ct];
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks) {
      const bf8 ak = frag(s.u.fe.k, 16 * wave + fr, 32 * ks + fk);
      gr[ct] = mfma(ak, frag(s.u.fe.k, 16 * ct + fr, 32 * ks + fk), gr[ct]);
      kq[ct] = mfma(ak, frag(s.u.fe.q, 16 * ct + fr, 32 * ks + fk), kq[ct]);
    }
  }
  {
    __bf16* wq = p.ws_q + gc * kChunkElems + lane * 8;
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks) {
      *reinterpret_cast<bf8*>(wq + (wave * 4 + ks) * kFrag) = frag(s.u.fe.q, 16 * wave + fr, 32 * ks + fk);
    }
    const int dk = tid & (kD - 1), ph = (tid >> 7) * 32;
#pragma unroll
    for (int q8 = 0; q8 < 4; ++q8) {
      bf8 v;
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = s.u.fe.k[ph + 8 * q8 + e][dk];
      *reinterpret_cast<bf8*>(&s.kt[dk][ph + 8 * q8]) = v;
    }
  }
  __syncthreads();
  {
    __bf16* wkt = p.ws_kt + gc * kChunkElems + lane * 8;
#pragma unroll
    for (int a2 = 0; a2 < 2; ++a2)
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int a = 2 * wave + a2;
        *reinterpret_cast<bf8*>(wkt + (a * 2 + ks) * kFrag) = frag(s.kt, 16 * a + fr, 32 * ks + fk);
      }
  }

  // ---- the k-head's v-heads, in groups of up to three ----
  const int rep_end = ONE_GROUP ? 1 : p.rep;
  for (int r0 = 0; r0 < rep_end; r0 += kGroup) {
    const int gs = min(kGroup, p.rep - r0);
    // gates and the in-chunk log decay (wave r: v-head r0 + r, lane = position)
    if (wave < gs) {
      const int h = g * p.rep + r0 + wave;
      const size_t hc = ((size_t)b * p.Hv + h) * p.nC + c;
      float al = 1.0f, be = 0.0f;  // padded steps: alpha 1, beta 0 (exact no-ops)
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
      s.G[wave][lane] = G;
      s.beta[wave][lane] = be;
      const float eg = d_expf(G);
      s.eG[wave][lane] = eg;
      const float Gl = __shfl(G, 63, 64);
      float* wg = p.ws_g + hc * kGStride;
      wg[lane] = eg;
      wg[64 + lane] = d_expf(Gl - G);
      if (lane == 0) wg[128] = d_expf(Gl);
    }
    __syncthreads();

    // A (into LDS as -A^T) and M (hi, lo to the workspace) from the registers
    for (int r = 0; r < gs; ++r) {
      const size_t hc = ((size_t)b * p.Hv + g * p.rep + r0 + r) * p.nC + c;
      __bf16* wm = p.ws_m + hc * kChunkElems;
      const int j0 = 16 * wave + 4 * lg;
      const f4 Gj = *reinterpret_cast<const f4*>(&s.G[r][j0]);
#pragma unroll
      for (int ct = 0; ct < 4; ++ct) {
        const int i = 16 * ct + fr;
        const float Gi = s.G[r][i], bi = s.beta[r][i];
        f4 mv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int j = j0 + e;
          const float dr = j <= i ? fast_exp(Gi - Gj[e]) : 0.0f;
          mv[e] = dr * kq[ct][e];
          s.u.nat[r][j][i] = j < i ? -((bi * dr) * gr[ct][e]) : 0.0f;
        }
        const bf4 hi = to_bf4(mv);
        const bf4 lo = to_bf4(mv - from_bf4(hi));
        // M row i, columns j0..j0+3; block (i / 16, j / 32), hi and lo blocks interleaved
        const int blk = ((i >> 4) * 2 + (j0 >> 5)) * 2;
        const int within = ((i & 15) + 16 * ((j0 & 31) >> 3)) * 8 + (j0 & 7);
        *reinterpret_cast<bf4*>(wm + blk * kFrag + within) = hi;
        *reinterpret_cast<bf4*>(wm + (blk + 1) * kFrag + within) = lo;
      }
    }
    __syncthreads();

    // T = (I + A)^-1: wave r inverts v-head r0 + r, lane j = column j, and writes T over
    // its own -A^T as [i][j] (only this wave has read that slot)
    if (wave < gs) {
      float x[kC];
      invert_column(s.u.nat[wave], lane, x);
#pragma unroll
      for (int i = 0; i < kC; ++i) s.u.nat[wave][i][lane] = x[i];
    }
    __syncthreads();

    for (int r = 0; r < gs; ++r) {
      const int h = g * p.rep + r0 + r;
      const size_t hc = ((size_t)b * p.Hv + h) * p.nC + c;
      // V: the B operand of U, straight from the workspace (a half chunk wholly past T was
      // never written: zeros)
      bf8 vb[kD / 16][2];
      {
        const __bf16* vf = p.ws_vf + hc * kChunkElems + lane * 8;
#pragma unroll
        for (int d = 0; d < kD / 16; ++d)
#pragma unroll
          for (int kh = 0; kh < 2; ++kh)
            vb[d][kh] = 32 * kh < n ? *reinterpret_cast<const bf8*>(vf + (2 * d + kh) * kFrag) : bf8{};
      }
      // column factors of T' = T diag(beta) and T' diag(e^G) for this lane's columns
      // j = 32 kh + fk + e
      float bj[2][8], ej[2][8];
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          bj[kh][e] = s.beta[r][32 * kh + fk + e];
          ej[kh][e] = s.eG[r][32 * kh + fk + e];
        }
      // U = T' V: wave w takes position tile w, all eight dv tiles; T' split into hi + lo
      {
        bf8 ah[2], al[2];
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          const float* xr = &s.u.nat[r][16 * wave + fr][32 * kh + fk];
          const f4 x0 = *reinterpret_cast<const f4*>(xr), x1 = *reinterpret_cast<const f4*>(xr + 4);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float tv = (e < 4 ? x0[e] : x1[e - 4]) * bj[kh][e];
            const __bf16 hi = (__bf16)tv;
            ah[kh][e] = hi;
            al[kh][e] = (__bf16)(tv - (float)hi);
          }
        }
        float* wu = p.ws_u + hc * kChunkElems + lane * 4;
#pragma unroll
        for (int d = 0; d < kD / 16; ++d) {
          f4 acc = {0.f, 0.f, 0.f, 0.f};
          acc = mfma(ah[0], vb[d][0], acc);
          acc = mfma(al[0], vb[d][0], acc);
          acc = mfma(ah[1], vb[d][1], acc);
          acc = mfma(al[1], vb[d][1], acc);
          *reinterpret_cast<f4*>(wu + (d * 4 + wave) * 256) = acc;
        }
      }
      // W^T = K^T (T' e^G)^T: wave w takes dk tiles 2w, 2w+1, all position tiles; lane
      // gets W[i = 16 bt + fr][dk = 16 a + 4 lg .. +3]
      {
        bf8 te[4][2];
#pragma unroll
        for (int bt = 0; bt < 4; ++bt)
#pragma unroll
          for (int kh = 0; kh < 2; ++kh) {
            const float* xr = &s.u.nat[r][16 * bt + fr][32 * kh + fk];
            const f4 x0 = *reinterpret_cast<const f4*>(xr), x1 = *reinterpret_cast<const f4*>(xr + 4);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              const float tv = (e < 4 ? x0[e] : x1[e - 4]) * bj[kh][e];
              te[bt][kh][e] = (__bf16)(tv * ej[kh][e]);
            }
          }
        __bf16* ww = p.ws_w + hc * kChunkElems;
#pragma unroll
        for (int a2 = 0; a2 < 2; ++a2) {
          const int a = 2 * wave + a2;
          const bf8 k0 = frag(s.kt, 16 * a + fr, fk), k1 = frag(s.kt, 16 * a + fr, 32 + fk);
#pragma unroll
          for (int bt = 0; bt < 4; ++bt) {
            f4 acc = {0.f, 0.f, 0.f, 0.f};
            acc = mfma(k0, te[bt][0], acc);
            acc = mfma(k1, te[bt][1], acc);
            *reinterpret_cast<bf4*>(ww + frag_off(16 * bt + fr, 16 * a + 4 * lg, kD / 32)) = to_bf4(acc);
          }
        }
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
  const int c = blockIdx.x % p.nC;
  const int rest = blockIdx.x / p.nC;
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
    const int dv = 16 * (f / 2) + (l & 15), pos = 32 * (f & 1) + 8 * (l >> 4);
    *reinterpret_cast<bf8*>(vf + e * 8) = *reinterpret_cast<const bf8*>(&vt[dv][pos]);
  }
}

// ============================================================================ scan

struct ScanSmem {
  __bf16 st[kDt][kD + kPadB];  // S^T (bf16): [dt][dk]
  __bf16 vh[kDt][kC + kPadB];  // V' hi: [dt][pos]
  __bf16 vl[kDt][kC + kPadB];  // V' lo
  __bf16 vp[kDt][kC + kPadB];  // e^(G63-G) V'
  float y[kC][kDt + 4];        // the chunk's outputs, written to o one chunk later
};

// The outputs staged in s.y for the chunk starting at t0 (n positions) to o: thread t
// stores positions t / 4, columns 8 (t % 4) .. +7 of the tile, 16 or 32 bytes.
__device__ __forceinline__ void store_outputs(const PrefillParams& p, const ScanSmem& s, int b, int h, int jt, int t0,
                                              int n, int tid) {
  const int pos = tid >> 2, c8 = (tid & 3) * 8;
  if (pos >= n) return;
  const f4 y0 = *reinterpret_cast<const f4*>(&s.y[pos][c8]);
  const f4 y1 = *reinterpret_cast<const f4*>(&s.y[pos][c8 + 4]);
  const size_t oi = (((size_t)b * p.T + t0 + pos) * p.Hv + h) * kD + jt * kDt + c8;
  if (p.o_bf16) {
    bf8 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = (__bf16)y0[e];
      v[4 + e] = (__bf16)y1[e];
    }
    *reinterpret_cast<bf8*>(static_cast<__bf16*>(p.o) + oi) = v;
  } else {
    *reinterpret_cast<f4*>(static_cast<float*>(p.o) + oi) = y0;
    *reinterpret_cast<f4*>(static_cast<float*>(p.o) + oi + 4) = y1;
  }
}

// One chunk's operands of one wave, in registers.
struct ChunkIn {
  bf8 q[4];       // Q rows 16w.., k = dk
  bf8 w[4];       // W rows 16w.., k = dk
  bf8 kt[2][2];   // K^T rows 32w + 16rt.., k = pos
  bf8 m[2][2];    // M rows 16w.., k = pos; [ks][hi, lo]
  f4 u[2];        // U (pos 16w + 4lg + e, dv 32jt + 16ct + fr)
  f4 eg, egr;     // e^G, e^(G63-G) at pos 16w + 4lg + e
  float gam;      // e^G63
};

// Part PART of one chunk's operands: 0 Q and the gate factors, 1 W, 2 M and U, 3 K^T.
// The parts are issued at different points of a chunk so that the memory pipeline is
// fed evenly and the wave is never held at a long run of loads.
template <int PART>
__device__ __forceinline__ void load_part(const PrefillParams& p, int b, int g, int h, int jt, int c, int wave,
                                          int lane, ChunkIn& in) {
  const size_t gc = ((size_t)b * p.Hk + g) * p.nC + c;
  const size_t hc = ((size_t)b * p.Hv + h) * p.nC + c;
  if (PART == 0) {
    const __bf16* q = p.ws_q + gc * kChunkElems + lane * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) in.q[ks] = *reinterpret_cast<const bf8*>(q + (wave * 4 + ks) * kFrag);
    const float* gg = p.ws_g + hc * kGStride + 16 * wave + 4 * (lane >> 4);
    in.eg = *reinterpret_cast<const f4*>(gg);
    in.egr = *reinterpret_cast<const f4*>(gg + 64);
    in.gam = p.ws_g[hc * kGStride + 128];
  } else if (PART == 1) {
    const __bf16* w = p.ws_w + hc * kChunkElems + lane * 8;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) in.w[ks] = *reinterpret_cast<const bf8*>(w + (wave * 4 + ks) * kFrag);
  } else if (PART == 2) {
    const __bf16* m = p.ws_m + hc * kChunkElems + lane * 8;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) in.m[i][j] = *reinterpret_cast<const bf8*>(m + ((wave * 2 + i) * 2 + j) * kFrag);
    const float* u = p.ws_u + hc * kChunkElems + lane * 4;
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) in.u[ct] = *reinterpret_cast<const f4*>(u + ((2 * jt + ct) * 4 + wave) * 256);
  } else {
    const __bf16* kt = p.ws_kt + gc * kChunkElems + lane * 8;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 2; ++j) in.kt[i][j] = *reinterpret_cast<const bf8*>(kt + ((2 * wave + i) * 2 + j) * kFrag);
  }
}

__device__ __forceinline__ void load_chunk(const PrefillParams& p, int b, int g, int h, int jt, int c, int wave,
                                           int lane, ChunkIn& in) {
  load_part<0>(p, b, g, h, jt, c, wave, lane, in);
  load_part<1>(p, b, g, h, jt, c, wave, lane, in);
  load_part<2>(p, b, g, h, jt, c, wave, lane, in);
  load_part<3>(p, b, g, h, jt, c, wave, lane, in);
}

// One chunk: uses `in`, loads chunk c + 2 (the last chunk again at the end) into `nx`.
__device__ __forceinline__ void scan_chunk(const PrefillParams& p, ScanSmem& s, f4 (&S)[2][2], const ChunkIn& in,
                                           ChunkIn& nx, int b, int g, int h, int jt, int c, int wave, int lane) {
  const int fr = lane & 15, fk = (lane >> 4) * 8, fq = (lane >> 4) * 4;
  // S^T in bf16 for the W S and Q S products
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct)
      *reinterpret_cast<bf4*>(&s.st[16 * ct + fr][32 * wave + 16 * rt + fq]) = to_bf4(S[rt][ct]);
  __syncthreads();
  const int cn = min(c + 2, p.nC - 1);
  load_part<0>(p, b, g, h, jt, cn, wave, lane, nx);
  __builtin_amdgcn_sched_barrier(0);
  // the previous chunk's outputs (staged before this chunk's first barrier)
  if (c > 0) store_outputs(p, s, b, h, jt, (c - 1) * kC, kC, threadIdx.x);

  // P = W S, QS = Q S (wave w: positions 16w..); V' = U - P
  f4 QS[2];
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    // the four S^T fragments in flight together, then the products (one LDS latency
    // instead of four: the register budget left the compiler no room to do it itself)
    bf8 bs[kD / 32];
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks) bs[ks] = frag(s.st, 16 * ct + fr, 32 * ks + fk);
    __builtin_amdgcn_sched_barrier(0);
    f4 P = {0.f, 0.f, 0.f, 0.f};
    QS[ct] = P;
#pragma unroll
    for (int ks = 0; ks < kD / 32; ++ks) {
      P = mfma(in.w[ks], bs[ks], P);
      QS[ct] = mfma(in.q[ks], bs[ks], QS[ct]);
    }
    const f4 vpr = in.u[ct] - P;
    const bf4 hi = to_bf4(vpr);
    *reinterpret_cast<bf4*>(&s.vh[16 * ct + fr][16 * wave + fq]) = hi;
    *reinterpret_cast<bf4*>(&s.vl[16 * ct + fr][16 * wave + fq]) = to_bf4(vpr - from_bf4(hi));
    *reinterpret_cast<bf4*>(&s.vp[16 * ct + fr][16 * wave + fq]) = to_bf4(in.egr * vpr);
    if (ct == 0) {
      __builtin_amdgcn_sched_barrier(0);
      load_part<1>(p, b, g, h, jt, cn, wave, lane, nx);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  __syncthreads();
  load_part<2>(p, b, g, h, jt, cn, wave, lane, nx);
  __builtin_amdgcn_sched_barrier(0);

  // y = e^G . QS + M V' (split operands), staged in LDS
#pragma unroll
  for (int ct = 0; ct < 2; ++ct) {
    bf8 bh[kC / 32], bl[kC / 32];  // V' hi and lo fragments in flight together
#pragma unroll
    for (int ks = 0; ks < kC / 32; ++ks) {
      bh[ks] = frag(s.vh, 16 * ct + fr, 32 * ks + fk);
      bl[ks] = frag(s.vl, 16 * ct + fr, 32 * ks + fk);
    }
    __builtin_amdgcn_sched_barrier(0);
    f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < kC / 32; ++ks) {
      acc = mfma(in.m[ks][0], bh[ks], acc);
      acc = mfma(in.m[ks][1], bh[ks], acc);
      acc = mfma(in.m[ks][0], bl[ks], acc);
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) s.y[16 * wave + fq + e][16 * ct + fr] = in.eg[e] * QS[ct][e] + acc[e];
  }

  // S = e^G63 S + K^T (e^(G63-G) V')
  __builtin_amdgcn_sched_barrier(0);
  load_part<3>(p, b, g, h, jt, cn, wave, lane, nx);
  __builtin_amdgcn_sched_barrier(0);
  bf8 bp[2][kC / 32];  // the four e^(G63-G) V' fragments in flight together
#pragma unroll
  for (int ct = 0; ct < 2; ++ct)
#pragma unroll
    for (int ks = 0; ks < kC / 32; ++ks) bp[ct][ks] = frag(s.vp, 16 * ct + fr, 32 * ks + fk);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      f4 acc = S[rt][ct] * in.gam;
#pragma unroll
      for (int ks = 0; ks < kC / 32; ++ks) acc = mfma(in.kt[rt][ks], bp[ct][ks], acc);
      S[rt][ct] = acc;
    }
}

__global__ __launch_bounds__(kThreads) void prefill_scan_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) ScanSmem s;
  // Workgroups are dispatched to the 8 XCDs round robin (bid % 8); renumber them so that
  // each XCD gets a contiguous range of (batch, v-head, tile) -- whole k-head groups when
  // the count divides -- and the chunk operands they share are fetched into one L2.
  int bid = blockIdx.x;
  if (gridDim.x % 8 == 0) bid = (bid & 7) * (gridDim.x >> 3) + (bid >> 3);
  const int jt = bid % (kD / kDt);
  const int rest = bid / (kD / kDt);
  const int h = rest % p.Hv;
  const int b = rest / p.Hv;
  const int g = h / p.rep;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int fr = lane & 15, fq = (lane >> 4) * 4;

  // S tile (Dk x 32) in accumulators: wave w holds dk rows 32w + 16rt + fq + e, dt 16ct + fr
  f4 S[2][2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      S[rt][ct] = f4{0.f, 0.f, 0.f, 0.f};
      if (p.state_in) {
        const float* sin = p.state_in + ((size_t)b * p.Hv + h) * kD * kD;
        S[rt][ct] = *reinterpret_cast<const f4*>(sin + (size_t)(jt * kDt + 16 * ct + fr) * kD + 32 * wave + 16 * rt + fq);
      }
    }

  // Operands are loaded two chunks ahead of their use (memory latency under this load
  // is longer than one chunk's work), in three register sets that rotate. The loop body
  // is three unconditional chunks and is only reached through three peeled ones, so it
  // is entered with the same loads in flight, in the same registers, as at its back
  // edge: the waits for a chunk's operands then never cover the loads issued after them.
  ChunkIn A, B, C;
  load_chunk(p, b, g, h, jt, 0, wave, lane, A);
  load_chunk(p, b, g, h, jt, min(1, p.nC - 1), wave, lane, B);
  if (p.nC < 3) {
    scan_chunk(p, s, S, A, C, b, g, h, jt, 0, wave, lane);
    if (p.nC > 1) scan_chunk(p, s, S, B, A, b, g, h, jt, 1, wave, lane);
  } else {
    scan_chunk(p, s, S, A, C, b, g, h, jt, 0, wave, lane);
    scan_chunk(p, s, S, B, A, b, g, h, jt, 1, wave, lane);
    scan_chunk(p, s, S, C, B, b, g, h, jt, 2, wave, lane);
    int c = 3;
    for (; c + 3 <= p.nC; c += 3) {
      scan_chunk(p, s, S, A, C, b, g, h, jt, c, wave, lane);
      scan_chunk(p, s, S, B, A, b, g, h, jt, c + 1, wave, lane);
      scan_chunk(p, s, S, C, B, b, g, h, jt, c + 2, wave, lane);
    }
    if (c < p.nC) scan_chunk(p, s, S, A, C, b, g, h, jt, c, wave, lane);
    if (c + 1 < p.nC) scan_chunk(p, s, S, B, A, b, g, h, jt, c + 1, wave, lane);
  }
  __syncthreads();
  store_outputs(p, s, b, h, jt, (p.nC - 1) * kC, p.T - (p.nC - 1) * kC, threadIdx.x);

  if (p.state_out) {
    float* sout = p.state_out + ((size_t)b * p.Hv + h) * kD * kD;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
        *reinterpret_cast<f4*>(sout + (size_t)(jt * kDt + 16 * ct + fr) * kD + 32 * wave + 16 * rt + fq) = S[rt][ct];
  }
}

struct WorkspaceLayout {
  size_t q, kt, w, m, u, g, vf, fq, fk, total;
};

// conv: the conv front end's bf16 q, k (B,T,Hk,128) are staged in the workspace too (its v
// goes to vf, which the qkv front end fills from the caller's v).
WorkspaceLayout workspace_layout(int B, int T, int Hk, int Hv, bool conv) {
  const size_t nC = (size_t)(T + kC - 1) / kC;
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t qk = al((size_t)B * Hk * nC * kChunkElems * 2);
  const size_t wm = al((size_t)B * Hv * nC * kChunkElems * 2);
  const size_t uu = al((size_t)B * Hv * nC * kChunkElems * 4);
  const size_t gg = al((size_t)B * Hv * nC * kGStride * 4);
  WorkspaceLayout L;
  L.q = 0;
  L.kt = L.q + qk;
  L.w = L.kt + qk;
  L.m = L.w + wm;
  L.u = L.m + wm;
  L.g = L.u + uu;
  const size_t fqk = conv ? al((size_t)B * T * Hk * kD * 2) : 0;
  L.vf = L.g + gg;
  L.fq = L.vf + wm;
  L.fk = L.fq + fqk;
  L.total = L.fk + fqk;
  return L;
}

}  // namespace

size_t prefill_workspace_bytes(int B, int T, int Hk, int Hv, bool conv) {
  return workspace_layout(B, T, Hk, Hv, conv).total;
}

hipError_t launch_chunked_prefill(const gdn_layer_args& a, void* workspace, hipStream_t stream) {
  PrefillParams p{};
  p.B = a.batch;
  p.T = a.seq_len;
  p.Hk = a.num_k_heads;
  p.Hv = a.num_v_heads;
  p.rep = p.Hv / p.Hk;
  p.C = 2 * p.Hk * kD + p.Hv * kD;
  p.nC = (p.T + kC - 1) / kC;
  p.gate_raw = a.gate_mode == GDN_GATES_RAW;
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
  const WorkspaceLayout L = workspace_layout(p.B, p.T, p.Hk, p.Hv, conv);
  char* w = static_cast<char*>(workspace);
  p.ws_q = reinterpret_cast<__bf16*>(w + L.q);
  p.ws_kt = reinterpret_cast<__bf16*>(w + L.kt);
  p.ws_w = reinterpret_cast<__bf16*>(w + L.w);
  p.ws_m = reinterpret_cast<__bf16*>(w + L.m);
  p.ws_u = reinterpret_cast<float*>(w + L.u);
  p.ws_g = reinterpret_cast<float*>(w + L.g);
  p.ws_vf = reinterpret_cast<__bf16*>(w + L.vf);
  if (conv) {
    p.q = reinterpret_cast<const __bf16*>(w + L.fq);
    p.k = reinterpret_cast<const __bf16*>(w + L.fk);
    p.v = nullptr;  // the front end writes v straight into ws_vf
  }

  const dim3 block(kThreads);
  const dim3 g1((unsigned)((size_t)p.B * p.Hk * p.nC));
  const dim3 g2((unsigned)((size_t)p.B * p.Hv * (kD / kDt)));
  if (conv) {
    const size_t nh = ((size_t)2 * p.Hk + p.Hv + kFeHeads - 1) / kFeHeads;
    const dim3 g0((unsigned)((size_t)p.B * ((p.T + kFePos - 1) / kFePos) * nh));
    hipLaunchKernelGGL(prefill_frontend_kernel, g0, block, 0, stream, p);
  } else {
    const dim3 gv((unsigned)((size_t)p.B * p.Hv * p.nC));
    hipLaunchKernelGGL(prefill_vfrag_kernel, gv, block, 0, stream, p);
  }
  if (p.rep <= kGroup) {
    hipLaunchKernelGGL((prefill_intra_kernel<true>), g1, block, 0, stream, p);
  } else {
    hipLaunchKernelGGL((prefill_intra_kernel<false>), g1, block, 0, stream, p);
  }
  hipLaunchKernelGGL(prefill_scan_kernel, g2, block, 0, stream, p);
  return hipGetLastError();
}

}  // namespace gdn
