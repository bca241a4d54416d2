// Chunked (WY / UT-transform) prefill of the gated-delta recurrence for gfx950, chunk 64.
//
// For one v-head and a chunk of positions i = 0..63 (python/qwen35.py:365-431):
//   G_i   = sum_{m<=i} log clip(alpha_m, 1e-6, 1)        (within-chunk log decay)
//   A_ij  = beta_i exp(G_i - G_j) (K K^T)_ij, j < i      T' = (I + A)^-1 diag(beta)
//   M_ij  = exp(G_i - G_j) (Q K^T)_ij, j <= i
// and, with the state S as (Dk x Dv) (the transpose of the stored (Dv, Dk) layout):
//   V' = T' (V - e^G . K S)                              (= U0 - Kt S of the reference)
//   y  = e^G . (Q S) + M V'                              (= MU0 + Qeff S)
//   S  = e^{G_63} S + K^T (e^{G_63 - G} . V')
//
// Two kernels:
//   prefill_intra  one workgroup per (batch, k-head, chunk), all chunks in parallel: the
//                  conv front end for q and k (or the given q, k), Q K^T and K K^T on bf16
//                  MFMA, and for each of the k-head's v-heads the gates, T' (blocked
//                  forward substitution in fp32) and M. Results go to the workspace.
//   prefill_scan   one workgroup per (batch, v-head, 32-column Dv tile), serial over the
//                  chunks; the fp32 state tile lives in MFMA accumulators. K S, Q S and
//                  K^T V' use bf16 operands; T' R and M V' split both operands into bf16
//                  hi + lo parts (three MFMAs), which keeps those two products -- the ones
//                  the output is most sensitive to -- at about fp32 accuracy.
//
// MFMA: v_mfma_f32_16x16x32_bf16. Lane l holds A[l%16][8(l/16)+i], B[8(l/16)+i][l%16]
// and C[4(l/16)+i][l%16] (i < 8, 8, 4). LDS matrices are stored so that both operands
// are read as 16-byte rows ([row][k] for A, [col][k] for B), padded by 8 bf16 per row to
// keep the 16 rows of a fragment on distinct banks.
#include "../../include/gdn.h"
#include "gdn_device_math.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

typedef __bf16 bf8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kC = 64;           // chunk
constexpr int kPadB = 8;         // bf16 padding per LDS row
constexpr int kDt = 32;          // Dv columns per scan workgroup
constexpr int kThreads = 256;
constexpr int kGStride = 132;    // floats per (v-head, chunk) in the gate workspace

__device__ __forceinline__ __bf16 to_bf(float x) { return __builtin_bit_cast(__bf16, f2bf(x)); }
__device__ __forceinline__ float from_bf(__bf16 x) { return bf2f(__builtin_bit_cast(uint16_t, x)); }

__device__ __forceinline__ f4 mfma(bf8 a, bf8 b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

template <int LD>
__device__ __forceinline__ bf8 frag(const __bf16 (*m)[LD], int row, int k) {
  return *reinterpret_cast<const bf8*>(&m[row][k]);
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
  // workspace
  __bf16* ws_q;   // (B, Hk, nC, 64, 128)
  __bf16* ws_k;   // (B, Hk, nC, 64, 128)
  __bf16* ws_kt;  // (B, Hk, nC, 128, 64)
  __bf16* ws_T;   // (B, Hv, nC, 2, 64, 64)  T' hi, lo
  __bf16* ws_M;   // (B, Hv, nC, 2, 64, 64)  M hi, lo
  float* ws_g;    // (B, Hv, nC, kGStride): e^G [64], e^(G63-G) [64], e^G63
};

// silu on a bf16 value: x * sigmoid(x), both ops rounded (ops.cpp:20).
__device__ __forceinline__ float silu_bf(float y) {
  const float sg = rbf(d_sigmoidf(y));
  return rbf(y * sg);
}

// Causal depthwise conv from 4 staged rows (model.cpp:385-395), bf16 after every op.
__device__ __forceinline__ float conv4_rows(float x0, float x1, float x2, float x3, const float (&w)[kTaps]) {
  float y = rbf(x0 * w[0]);
  y = rbf(y + rbf(x1 * w[1]));
  y = rbf(y + rbf(x2 * w[2]));
  y = rbf(y + rbf(x3 * w[3]));
  return y;
}

__device__ __forceinline__ float wave64_sum(float x) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) x = x + __shfl_xor(x, m, 64);
  return x;
}

// Padded conv input row `pos` (absolute position; negative rows come from the conv
// state) at channel c; 0 past the end of the sequence.
__device__ __forceinline__ uint16_t xp_row(const PrefillParams& p, int b, int pos, int c) {
  if (pos >= p.T) return 0;
  if (pos < 0) {
    return p.conv_in ? p.conv_in[((size_t)b * kConvRows + (kConvRows + pos)) * p.C + c] : (uint16_t)0;
  }
  return p.x[((size_t)b * p.T + pos) * p.C + c];
}

typedef uint16_t u16x8 __attribute__((ext_vector_type(8)));

// Eight consecutive channels of padded conv input row `pos` (16-byte aligned: C and the
// channel offset are multiples of 8, x and the conv state 16-byte aligned).
__device__ __forceinline__ u16x8 xp_vec8(const PrefillParams& p, int b, int pos, int c) {
  if (pos >= p.T) return u16x8{};
  if (pos < 0) {
    if (!p.conv_in) return u16x8{};
    return *reinterpret_cast<const u16x8*>(p.conv_in + ((size_t)b * kConvRows + (kConvRows + pos)) * p.C + c);
  }
  return *reinterpret_cast<const u16x8*>(p.x + ((size_t)b * p.T + pos) * p.C + c);
}

// ============================================================================ intra

struct IntraSmem {
  __bf16 q[kC][kD + kPadB];
  __bf16 k[kC][kD + kPadB];
  float gram[kC][kC + 4];
  float qk[kC][kC + 4];
  union {
    uint16_t xs[kC + kConvRows][2 * kD];  // staged conv input rows (front end only)
    struct {
      float a[kC][kC + 4];
      float t[kC][kC + 4];
    } m;
  } u;
  float tmp[4][16][17];
  float G[kC];
  float beta[kC];
};

// One off-diagonal 16x16 block of T = (I + A)^-1 (block rows i > j), by one wave:
// X_ij = -X_ii sum_{m=j}^{i-1} A_im X_mj. Lane l computes rows 4(l/16)..+3, column l%16.
__device__ __forceinline__ void inverse_offdiag(IntraSmem& s, int bi, int bj, int wave, int lane) {
  const int col = lane & 15, r0 = (lane >> 4) * 4;
  float y[4] = {0.f, 0.f, 0.f, 0.f};
  for (int bm = bj; bm < bi; ++bm) {
    for (int m = 0; m < 16; ++m) {
      const float xv = s.u.m.t[16 * bm + m][16 * bj + col];
#pragma unroll
      for (int r = 0; r < 4; ++r) y[r] = __builtin_fmaf(s.u.m.a[16 * bi + r0 + r][16 * bm + m], xv, y[r]);
    }
  }
  float(*tmp)[17] = s.tmp[wave];
#pragma unroll
  for (int r = 0; r < 4; ++r) tmp[r0 + r][col] = y[r];
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  float z[4] = {0.f, 0.f, 0.f, 0.f};
  for (int m = 0; m < 16; ++m) {
    const float yv = tmp[m][col];
#pragma unroll
    for (int r = 0; r < 4; ++r) z[r] = __builtin_fmaf(s.u.m.t[16 * bi + r0 + r][16 * bi + m], yv, z[r]);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) s.u.m.t[16 * bi + r0 + r][16 * bj + col] = -z[r];
}

template <int FE>
__global__ __launch_bounds__(kThreads) void prefill_intra_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) IntraSmem s;
  const int c = blockIdx.x % p.nC;
  int rest = blockIdx.x / p.nC;
  const int g = rest % p.Hk;
  const int b = rest / p.Hk;
  const int t0 = c * kC;
  const int n = min(kC, p.T - t0);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

  // ---- q, k of the chunk into LDS (bf16) ----
  if (FE == 1) {
    // stage rows t0-3 .. t0+63 of the q and k channels of k-head g: 16-byte loads, all
    // issued before any is used
    {
      constexpr int kVec = (kC + kConvRows) * 2 * kD / 8;  // 16-byte pieces
      constexpr int kIter = (kVec + kThreads - 1) / kThreads;
      u16x8 vals[kIter];
#pragma unroll
      for (int it = 0; it < kIter; ++it) {
        const int e = tid + it * kThreads;
        const int r = e / (2 * kD / 8), cc = (e % (2 * kD / 8)) * 8;
        const int ch = (cc < kD ? 0 : p.Hk * kD - kD) + g * kD + cc;
        vals[it] = e < kVec ? xp_vec8(p, b, t0 - kConvRows + r, ch) : u16x8{};
      }
#pragma unroll
      for (int it = 0; it < kIter; ++it) {
        const int e = tid + it * kThreads;
        if (e < kVec) {
          const int r = e / (2 * kD / 8), cc = (e % (2 * kD / 8)) * 8;
          *reinterpret_cast<u16x8*>(&s.u.xs[r][cc]) = vals[it];
        }
      }
    }
    __syncthreads();
    // wave 0/1: q of positions 0..31 / 32..63; wave 2/3: k. Lane: channels l, l+64.
    const int part = wave >> 1;
    const int pbase = (wave & 1) * 32;
    const uint16_t* w_l = p.conv_w;
    float w0[kTaps], w1[kTaps];
    const int ch0 = part * p.Hk * kD + g * kD + lane;
#pragma unroll
    for (int j = 0; j < kTaps; ++j) {
      w0[j] = bf2f(w_l[(size_t)j * p.C + ch0]);
      w1[j] = bf2f(w_l[(size_t)j * p.C + ch0 + 64]);
    }
    __bf16(*dst)[kD + kPadB] = part == 0 ? s.q : s.k;
    const int col = part * kD + lane;
    for (int pp = 0; pp < 32; ++pp) {
      const int pos = pbase + pp;
      float y0 = 0.f, y1 = 0.f;
      if (pos < n) {
        const float u0 = silu_bf(conv4_rows(bf2f(s.u.xs[pos][col]), bf2f(s.u.xs[pos + 1][col]),
                                            bf2f(s.u.xs[pos + 2][col]), bf2f(s.u.xs[pos + 3][col]), w0));
        const float u1 = silu_bf(conv4_rows(bf2f(s.u.xs[pos][col + 64]), bf2f(s.u.xs[pos + 1][col + 64]),
                                            bf2f(s.u.xs[pos + 2][col + 64]), bf2f(s.u.xs[pos + 3][col + 64]), w1));
        // l2norm (ops.cpp:27-30) with the butterfly sum order of the decode path
        const float scale_b = rbf(1.0f / sqrtf((float)kD));
        const float eps_b = rbf(1e-6f);
        const float pr = rbf(u0 * u0) + rbf(u1 * u1);
        const float ssum = rbf(wave64_sum(pr));
        const float den = rbf(ssum + eps_b);
        const float rs = rbf(1.0f / sqrtf(den));
        y0 = rbf(u0 * rs);
        y1 = rbf(u1 * rs);
        if (part == 0) {
          y0 = rbf(y0 * scale_b);
          y1 = rbf(y1 * scale_b);
        }
      }
      dst[pos][lane] = to_bf(y0);
      dst[pos][lane + 64] = to_bf(y1);
    }
    // the conv state hand-off: rows T..T+2 of [conv_in ; x], written by the last
    // chunk's workgroup of each k-head for its q, k and v channels
    if (p.conv_out && c == p.nC - 1) {
      const int nch = 2 * kD + p.rep * kD;
      for (int e = tid; e < nch * kConvRows; e += kThreads) {
        const int r = e / nch, cc = e % nch;
        const int ch = cc < kD ? g * kD + cc
                     : cc < 2 * kD ? p.Hk * kD + g * kD + (cc - kD)
                                   : 2 * p.Hk * kD + g * p.rep * kD + (cc - 2 * kD);
        p.conv_out[((size_t)b * kConvRows + r) * p.C + ch] = xp_row(p, b, p.T - kConvRows + r, ch);
      }
    }
  } else {
    for (int e = tid; e < kC * kD; e += kThreads) {
      const int pos = e / kD, d = e % kD;
      __bf16 qv = to_bf(0.f), kv = to_bf(0.f);
      if (pos < n) {
        const size_t gi = (((size_t)b * p.T + t0 + pos) * p.Hk + g) * kD + d;
        qv = p.q[gi];
        kv = p.k[gi];
      }
      s.q[pos][d] = qv;
      s.k[pos][d] = kv;
    }
  }
  __syncthreads();

  // ---- q, k, k^T to the workspace ----
  {
    const size_t base = (((size_t)b * p.Hk + g) * p.nC + c) * kC * kD;
    for (int e = tid; e < kC * kD / 8; e += kThreads) {
      const int pos = e / (kD / 8), d8 = (e % (kD / 8)) * 8;
      *reinterpret_cast<bf8*>(p.ws_q + base + pos * kD + d8) = frag(s.q, pos, d8);
      *reinterpret_cast<bf8*>(p.ws_k + base + pos * kD + d8) = frag(s.k, pos, d8);
    }
    for (int e = tid; e < kC * kD; e += kThreads) {
      const int d = e / kC, pos = e % kC;
      p.ws_kt[base + (size_t)d * kC + pos] = s.k[pos][d];
    }
  }

  // ---- K K^T and Q K^T (64 x 64) on MFMA: wave w takes row tile w ----
  {
    const int fr = lane & 15, fk = (lane >> 4) * 8;
#pragma unroll
    for (int ct = 0; ct < 4; ++ct) {
      f4 ag = {0.f, 0.f, 0.f, 0.f}, aq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kD / 32; ++ks) {
        const bf8 bk = frag(s.k, 16 * ct + fr, 32 * ks + fk);
        ag = mfma(frag(s.k, 16 * wave + fr, 32 * ks + fk), bk, ag);
        aq = mfma(frag(s.q, 16 * wave + fr, 32 * ks + fk), bk, aq);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s.gram[16 * wave + (lane >> 4) * 4 + i][16 * ct + fr] = ag[i];
        s.qk[16 * wave + (lane >> 4) * 4 + i][16 * ct + fr] = aq[i];
      }
    }
  }
  __syncthreads();

  // ---- per v-head: gates, T', M ----
  for (int r = 0; r < p.rep; ++r) {
    const int h = g * p.rep + r;
    const size_t hc = ((size_t)b * p.Hv + h) * p.nC + c;
    if (wave == 0) {
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
      // inclusive prefix sum over the 64 lanes (positions)
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float up = __shfl_up(G, off, 64);
        if (lane >= off) G = G + up;
      }
      s.G[lane] = G;
      s.beta[lane] = be;
      const float Gl = __shfl(G, 63, 64);
      float* wg = p.ws_g + hc * kGStride;
      wg[lane] = d_expf(G);
      wg[64 + lane] = d_expf(Gl - G);
      if (lane == 0) wg[128] = d_expf(Gl);
    }
    __syncthreads();
    // A (strictly lower) and M (lower incl. diagonal)
    __bf16* wm = p.ws_M + hc * 2 * kC * kC;
    for (int e = tid; e < kC * kC; e += kThreads) {
      const int i = e / kC, j = e % kC;
      float av = 0.f, mv = 0.f;
      if (j <= i) {
        const float dr = d_expf(s.G[i] - s.G[j]);
        mv = dr * s.qk[i][j];
        if (j < i) av = s.beta[i] * dr * s.gram[i][j];
      }
      s.u.m.a[i][j] = av;
      s.u.m.t[i][j] = 0.f;
      const __bf16 hi = to_bf(mv);
      wm[e] = hi;
      wm[kC * kC + e] = to_bf(mv - from_bf(hi));
    }
    __syncthreads();
    // T = (I + A)^-1: diagonal 16x16 blocks by forward substitution (wave w, block w;
    // lane = column), then the off-diagonal blocks by block distance
    if (lane < 16) {
      const int o = 16 * wave;
      float xcol[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float v = (i == lane) ? 1.0f : 0.0f;
#pragma unroll
        for (int m = 0; m < i; ++m) v = __builtin_fmaf(-s.u.m.a[o + i][o + m], xcol[m], v);
        xcol[i] = v;
      }
#pragma unroll
      for (int i = 0; i < 16; ++i) s.u.m.t[o + i][o + lane] = xcol[i];
    }
    __syncthreads();
    if (wave < 3) inverse_offdiag(s, wave + 1, wave, wave, lane);
    __syncthreads();
    if (wave < 2) inverse_offdiag(s, wave + 2, wave, wave, lane);
    __syncthreads();
    if (wave == 0) inverse_offdiag(s, 3, 0, wave, lane);
    __syncthreads();
    // T' = T diag(beta), split into bf16 hi + lo
    __bf16* wt = p.ws_T + hc * 2 * kC * kC;
    for (int e = tid; e < kC * kC; e += kThreads) {
      const int i = e / kC, j = e % kC;
      const float tv = s.u.m.t[i][j] * s.beta[j];
      const __bf16 hi = to_bf(tv);
      wt[e] = hi;
      wt[kC * kC + e] = to_bf(tv - from_bf(hi));
    }
    __syncthreads();
  }
}

// ============================================================================ scan

struct ScanSmem {
  __bf16 q[kC][kD + kPadB];
  __bf16 k[kC][kD + kPadB];
  __bf16 kt[kD][kC + kPadB];
  __bf16 th[kC][kC + kPadB];
  __bf16 tl[kC][kC + kPadB];
  __bf16 mh[kC][kC + kPadB];
  __bf16 ml[kC][kC + kPadB];
  __bf16 st[kDt][kD + kPadB];    // S^T (bf16): [dt][dk]
  __bf16 rh[kDt][kC + kPadB];    // R: [dt][pos]
  __bf16 rl[kDt][kC + kPadB];
  __bf16 vph[kDt][kC + kPadB];   // V'
  __bf16 vpl[kDt][kC + kPadB];
  __bf16 vpp[kDt][kC + kPadB];   // e^(G63-G) V'
  float v[kC][kDt + 1];
  float eg[kC];
  float egr[kC];
  uint16_t xs[kC + kConvRows][kDt];  // 64-byte rows, 16-byte aligned
  float gam;
};

template <int FE>
__global__ __launch_bounds__(kThreads) void prefill_scan_kernel(PrefillParams p) {
  __shared__ __attribute__((aligned(16))) ScanSmem s;
  const int jt = blockIdx.x % (kD / kDt);
  int rest = blockIdx.x / (kD / kDt);
  const int h = rest % p.Hv;
  const int b = rest / p.Hv;
  const int g = h / p.rep;
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int fr = lane & 15, fk = (lane >> 4) * 8, fq = (lane >> 4) * 4;
  const int vch0 = 2 * p.Hk * kD + h * kD + jt * kDt;  // first v channel of the tile

  // S tile (Dk x 32) in accumulators: wave w holds dk rows 32w + 16rt + fq + i, dt 16ct + fr
  f4 S[2][2];
  {
    const float* sin = p.state_in ? p.state_in + ((size_t)b * p.Hv + h) * kD * kD : nullptr;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int dk = 32 * wave + 16 * rt + fq + i, dt = 16 * ct + fr;
          S[rt][ct][i] = sin ? sin[(size_t)(jt * kDt + dt) * kD + dk] : 0.0f;
        }
  }
  float wv[kTaps] = {};
  if (FE == 1) {
    const int dt = tid & (kDt - 1);
#pragma unroll
    for (int j = 0; j < kTaps; ++j) wv[j] = bf2f(p.conv_w[(size_t)j * p.C + vch0 + dt]);
  }

  for (int c = 0; c < p.nC; ++c) {
    const int t0 = c * kC;
    const int n = min(kC, p.T - t0);
    const size_t gc = ((size_t)b * p.Hk + g) * p.nC + c;
    const size_t hc = ((size_t)b * p.Hv + h) * p.nC + c;

    // ---- stage the chunk: every 16-byte load issued before any is stored ----
    {
      constexpr int kQK = kC * kD / 8 / kThreads;  // 4 pieces per thread per matrix
      constexpr int kTM = kC * kC / 8 / kThreads;  // 2
      bf8 vq[kQK], vk[kQK], vkt[kQK], vth[kTM], vtl[kTM], vmh[kTM], vml[kTM];
      const __bf16* wq = p.ws_q + gc * kC * kD;
      const __bf16* wk = p.ws_k + gc * kC * kD;
      const __bf16* wkt = p.ws_kt + gc * kC * kD;
      const __bf16* wt = p.ws_T + hc * 2 * kC * kC;
      const __bf16* wm = p.ws_M + hc * 2 * kC * kC;
#pragma unroll
      for (int it = 0; it < kQK; ++it) {
        const int e = tid + it * kThreads;
        vq[it] = *reinterpret_cast<const bf8*>(wq + e * 8);
        vk[it] = *reinterpret_cast<const bf8*>(wk + e * 8);
        vkt[it] = *reinterpret_cast<const bf8*>(wkt + e * 8);
      }
#pragma unroll
      for (int it = 0; it < kTM; ++it) {
        const int e = tid + it * kThreads;
        vth[it] = *reinterpret_cast<const bf8*>(wt + e * 8);
        vtl[it] = *reinterpret_cast<const bf8*>(wt + kC * kC + e * 8);
        vmh[it] = *reinterpret_cast<const bf8*>(wm + e * 8);
        vml[it] = *reinterpret_cast<const bf8*>(wm + kC * kC + e * 8);
      }
      float gv = 0.f, grv = 0.f, gam = 0.f;
      const float* wg = p.ws_g + hc * kGStride;
      if (tid < kC) {
        gv = wg[tid];
        grv = wg[64 + tid];
        gam = wg[128];
      }
      u16x8 xv[2] = {};
      constexpr int kXV = (kC + kConvRows) * kDt / 8;  // 268 pieces
      if (FE == 1) {
#pragma unroll
        for (int it = 0; it < 2; ++it) {
          const int e = tid + it * kThreads;
          if (e < kXV) xv[it] = xp_vec8(p, b, t0 - kConvRows + e / (kDt / 8), vch0 + (e % (kDt / 8)) * 8);
        }
      }
#pragma unroll
      for (int it = 0; it < kQK; ++it) {
        const int e = tid + it * kThreads;
        *reinterpret_cast<bf8*>(&s.q[e / (kD / 8)][(e % (kD / 8)) * 8]) = vq[it];
        *reinterpret_cast<bf8*>(&s.k[e / (kD / 8)][(e % (kD / 8)) * 8]) = vk[it];
        *reinterpret_cast<bf8*>(&s.kt[e / (kC / 8)][(e % (kC / 8)) * 8]) = vkt[it];
      }
#pragma unroll
      for (int it = 0; it < kTM; ++it) {
        const int e = tid + it * kThreads, i = e / (kC / 8), j8 = (e % (kC / 8)) * 8;
        *reinterpret_cast<bf8*>(&s.th[i][j8]) = vth[it];
        *reinterpret_cast<bf8*>(&s.tl[i][j8]) = vtl[it];
        *reinterpret_cast<bf8*>(&s.mh[i][j8]) = vmh[it];
        *reinterpret_cast<bf8*>(&s.ml[i][j8]) = vml[it];
      }
      if (tid < kC) {
        s.eg[tid] = gv;
        s.egr[tid] = grv;
        if (tid == 0) s.gam = gam;
      }
      if (FE == 1) {
#pragma unroll
        for (int it = 0; it < 2; ++it) {
          const int e = tid + it * kThreads;
          if (e < kXV) *reinterpret_cast<u16x8*>(&s.xs[e / (kDt / 8)][(e % (kDt / 8)) * 8]) = xv[it];
        }
      }
    }
    if (FE == 1) {
    } else {
      for (int e = tid; e < kC * kDt; e += kThreads) {
        const int pos = e / kDt, dt = e % kDt;
        s.v[pos][dt] = pos < n ? from_bf(p.v[(((size_t)b * p.T + t0 + pos) * p.Hv + h) * kD + jt * kDt + dt]) : 0.0f;
      }
    }
    // S^T in bf16 for the K S and Q S products
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) s.st[16 * ct + fr][32 * wave + 16 * rt + fq + i] = to_bf(S[rt][ct][i]);
    __syncthreads();
    if (FE == 1) {
      // v = silu(conv(x)) for the tile's 32 channels (bf16 values)
      const int dt = tid & (kDt - 1);
      for (int pos = tid / kDt; pos < kC; pos += kThreads / kDt) {
        float val = 0.f;
        if (pos < n) {
          val = silu_bf(conv4_rows(bf2f(s.xs[pos][dt]), bf2f(s.xs[pos + 1][dt]), bf2f(s.xs[pos + 2][dt]),
                                   bf2f(s.xs[pos + 3][dt]), wv));
        }
        s.v[pos][dt] = val;
      }
      __syncthreads();
    }

    // ---- P = K S, QS = Q S (64 x 32): wave w takes position rows 16w.. ----
    f4 QS[2];
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      f4 P = {0.f, 0.f, 0.f, 0.f};
      QS[ct] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kD / 32; ++ks) {
        const bf8 bs = frag(s.st, 16 * ct + fr, 32 * ks + fk);
        P = mfma(frag(s.k, 16 * wave + fr, 32 * ks + fk), bs, P);
        QS[ct] = mfma(frag(s.q, 16 * wave + fr, 32 * ks + fk), bs, QS[ct]);
      }
      // R = V - e^G . P, split into hi + lo, stored [dt][pos]
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pos = 16 * wave + fq + i, dt = 16 * ct + fr;
        const float rv = s.v[pos][dt] - s.eg[pos] * P[i];
        const __bf16 hi = to_bf(rv);
        s.rh[dt][pos] = hi;
        s.rl[dt][pos] = to_bf(rv - from_bf(hi));
      }
    }
    __syncthreads();

    // ---- V' = T' R (split operands) ----
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kC / 32; ++ks) {
        const bf8 ah = frag(s.th, 16 * wave + fr, 32 * ks + fk);
        const bf8 al = frag(s.tl, 16 * wave + fr, 32 * ks + fk);
        const bf8 bh = frag(s.rh, 16 * ct + fr, 32 * ks + fk);
        const bf8 bl = frag(s.rl, 16 * ct + fr, 32 * ks + fk);
        acc = mfma(ah, bh, acc);
        acc = mfma(al, bh, acc);
        acc = mfma(ah, bl, acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pos = 16 * wave + fq + i, dt = 16 * ct + fr;
        const __bf16 hi = to_bf(acc[i]);
        s.vph[dt][pos] = hi;
        s.vpl[dt][pos] = to_bf(acc[i] - from_bf(hi));
        s.vpp[dt][pos] = to_bf(s.egr[pos] * acc[i]);
      }
    }
    __syncthreads();

    // ---- y = e^G . QS + M V' (split operands) ----
#pragma unroll
    for (int ct = 0; ct < 2; ++ct) {
      f4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < kC / 32; ++ks) {
        const bf8 ah = frag(s.mh, 16 * wave + fr, 32 * ks + fk);
        const bf8 al = frag(s.ml, 16 * wave + fr, 32 * ks + fk);
        const bf8 bh = frag(s.vph, 16 * ct + fr, 32 * ks + fk);
        const bf8 bl = frag(s.vpl, 16 * ct + fr, 32 * ks + fk);
        acc = mfma(ah, bh, acc);
        acc = mfma(al, bh, acc);
        acc = mfma(ah, bl, acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int pos = 16 * wave + fq + i, dt = 16 * ct + fr;
        if (pos < n) {
          const float y = s.eg[pos] * QS[ct][i] + acc[i];
          const size_t oi = (((size_t)b * p.T + t0 + pos) * p.Hv + h) * kD + jt * kDt + dt;
          if (p.o_bf16) {
            static_cast<uint16_t*>(p.o)[oi] = f2bf(y);
          } else {
            static_cast<float*>(p.o)[oi] = y;
          }
        }
      }
    }

    // ---- S = e^G63 S + K^T (e^(G63-G) V') ----
    const float gam = s.gam;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        f4 acc = S[rt][ct] * gam;
#pragma unroll
        for (int ks = 0; ks < kC / 32; ++ks) {
          acc = mfma(frag(s.kt, 32 * wave + 16 * rt + fr, 32 * ks + fk), frag(s.vpp, 16 * ct + fr, 32 * ks + fk), acc);
        }
        S[rt][ct] = acc;
      }
    __syncthreads();
  }

  if (p.state_out) {
    float* sout = p.state_out + ((size_t)b * p.Hv + h) * kD * kD;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int dk = 32 * wave + 16 * rt + fq + i, dt = 16 * ct + fr;
          sout[(size_t)(jt * kDt + dt) * kD + dk] = S[rt][ct][i];
        }
  }
}

}  // namespace

size_t prefill_workspace_bytes(int B, int T, int Hk, int Hv) {
  const size_t nC = (size_t)(T + kC - 1) / kC;
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t qk = al((size_t)B * Hk * nC * kC * kD * 2);
  const size_t tm = al((size_t)B * Hv * nC * 2 * kC * kC * 2);
  const size_t gg = al((size_t)B * Hv * nC * kGStride * 4);
  return 3 * qk + 2 * tm + gg;
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
  auto al = [](size_t x) { return (x + 255) / 256 * 256; };
  const size_t nC = p.nC;
  char* w = static_cast<char*>(workspace);
  const size_t qk = al((size_t)p.B * p.Hk * nC * kC * kD * 2);
  const size_t tm = al((size_t)p.B * p.Hv * nC * 2 * kC * kC * 2);
  p.ws_q = reinterpret_cast<__bf16*>(w);
  p.ws_k = reinterpret_cast<__bf16*>(w + qk);
  p.ws_kt = reinterpret_cast<__bf16*>(w + 2 * qk);
  p.ws_T = reinterpret_cast<__bf16*>(w + 3 * qk);
  p.ws_M = reinterpret_cast<__bf16*>(w + 3 * qk + tm);
  p.ws_g = reinterpret_cast<float*>(w + 3 * qk + 2 * tm);

  const dim3 block(kThreads);
  const dim3 g1((unsigned)((size_t)p.B * p.Hk * p.nC));
  const dim3 g2((unsigned)((size_t)p.B * p.Hv * (kD / kDt)));
  if (a.frontend == GDN_FRONTEND_CONV) {
    hipLaunchKernelGGL((prefill_intra_kernel<1>), g1, block, 0, stream, p);
    hipLaunchKernelGGL((prefill_scan_kernel<1>), g2, block, 0, stream, p);
  } else {
    hipLaunchKernelGGL((prefill_intra_kernel<0>), g1, block, 0, stream, p);
    hipLaunchKernelGGL((prefill_scan_kernel<0>), g2, block, 0, stream, p);
  }
  return hipGetLastError();
}

}  // namespace gdn
