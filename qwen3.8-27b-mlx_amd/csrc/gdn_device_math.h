// Device-side scalar math for the gated-delta front end and gates (gfx950).
//
// The front end rounds to bf16 after every op (the reference's bf16 MLX ops,
// cpp/src/model.cpp:585-602, cpp/src/ops.cpp:20-30), so a one-ulp difference in an
// fp32 intermediate can flip a bf16 rounding and move an output by 2^-8 relative.
// To make those decisions reproducible, exp/log/log1p here are fixed algorithms built
// only from correctly rounded IEEE operations (add, mul, fma, div, sqrt, rint):
//   exp   Cody-Waite reduction x = n ln2 + r, |r| <= ln2/2; degree-7 Taylor polynomial
//         of e^r by Horner with fma; 2^n applied in two halves.
//   log   x = m 2^e, m in [sqrt(1/2), sqrt(2)), f = m - 1, s = f/(2+f):
//         log(1+f) = f - (f^2/2 - s (f^2/2 + R(s^2))), R the atanh series through s^8.
//   log1p Goldberg's correction log(w) * (x / (w - 1)), w = 1 + x.
// The translation unit is compiled with -ffp-contract=off, so every operation below is
// rounded exactly as written.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gdn {

__device__ __forceinline__ float bits_f(uint32_t u) { return __builtin_bit_cast(float, u); }
__device__ __forceinline__ uint32_t f_bits(float x) { return __builtin_bit_cast(uint32_t, x); }

// fp32 -> bf16 bits, round to nearest even, NaN quieted: one v_cvt_pk_bf16_f32. On
// gfx950 this instruction equals the integer rounding (u + 0x7fff + ((u >> 16) & 1)) >> 16,
// with NaN -> (u >> 16) | 0x40, for every one of the 2^32 fp32 inputs (checked
// exhaustively on the device).
__device__ __forceinline__ uint16_t f2bf(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }
__device__ __forceinline__ float bf2f(uint16_t h) { return bits_f((uint32_t)h << 16); }

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

// Round an fp32 value to the nearest bf16 value, kept in fp32: the pair (0, x) packs to
// bf16(x) << 16 | bf16(0), which is that value's fp32 bit pattern (one instruction).
__device__ __forceinline__ float rbf(float x) {
  return __builtin_bit_cast(float, __builtin_convertvector((f32x2_t){0.0f, x}, bf16x2_t));
}

// The special cases (NaN, overflow, underflow) are applied by select after the
// polynomial path has run on an argument clamped into range, so the function has no
// branches; for in-range arguments the clamp is the identity and every op is as listed.
__device__ __forceinline__ float d_expf(float x) {
  const float xc = __builtin_fminf(__builtin_fmaxf(x, -104.0f), 89.0f);
  const float n = __builtin_rintf(xc * 1.44269502162933349609375f);
  float r = __builtin_fmaf(-n, 0.693145751953125f, xc);
  r = __builtin_fmaf(-n, 1.428606765330187045e-06f, r);
  float p = 1.98412698412698412698e-4f;
  p = __builtin_fmaf(p, r, 1.38888888888888888889e-3f);
  p = __builtin_fmaf(p, r, 8.33333333333333333333e-3f);
  p = __builtin_fmaf(p, r, 4.16666666666666666667e-2f);
  p = __builtin_fmaf(p, r, 1.66666666666666666667e-1f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const int n1 = ni / 2, n2 = ni - n1;
  p = p * bits_f((uint32_t)(n1 + 127) << 23);
  float y = p * bits_f((uint32_t)(n2 + 127) << 23);
  y = x > 88.72283935546875f ? __builtin_inff() : y;
  y = x < -103.97208404541015625f ? 0.0f : y;
  return x != x ? x : y;
}

// log of a positive normal argument (the only arguments used here are in (1, 2]).
__device__ __forceinline__ float d_logf(float x) {
  uint32_t u = f_bits(x);
  int e = (int)((u >> 23) & 0xffu) - 127;
  float m = bits_f((u & 0x007fffffu) | 0x3f800000u);
  if (m > 1.41421356237309504880f) {
    m = m * 0.5f;
    e += 1;
  }
  const float f = m - 1.0f;
  const float s = f / (2.0f + f);
  const float z = s * s;
  float R = 0.22222222222222222222f;
  R = __builtin_fmaf(R, z, 0.28571428571428571429f);
  R = __builtin_fmaf(R, z, 0.4f);
  R = __builtin_fmaf(R, z, 0.66666666666666666667f);
  R = R * z;
  const float hfsq = 0.5f * f * f;
  const float lm = f - (hfsq - s * (hfsq + R));
  const float ef = (float)e;
  return __builtin_fmaf(ef, 0.693145751953125f, __builtin_fmaf(ef, 1.428606765330187045e-06f, lm));
}

__device__ __forceinline__ float d_log1pf(float x) {
  const float w = 1.0f + x;
  if (w == 1.0f) return x;
  if (w == __builtin_inff()) return w;
  return d_logf(w) * (x / (w - 1.0f));
}

// sigmoid(x) = 1 / (1 + exp(-x)), as MLX's unary op.
__device__ __forceinline__ float d_sigmoidf(float x) {
  const float e = d_expf(-x);
  const float d = 1.0f + e;
  return 1.0f / d;
}

// softplus(x) = logaddexp(0, x) (cpp/src/ops.cpp:22-25).
__device__ __forceinline__ float d_softplusf(float x) {
  if (x != x) return x;
  const float mx = x > 0.0f ? x : 0.0f;
  const float mn = x > 0.0f ? 0.0f : x;
  if (mn == -__builtin_inff() || mx == __builtin_inff()) return mx;
  return mx + d_log1pf(d_expf(mn - mx));
}

// silu on a bf16 value: x * sigmoid(x), both ops rounded (cpp/src/ops.cpp:20).
__device__ __forceinline__ float silu_bf(float y) {
  const float sg = rbf(d_sigmoidf(y));
  return rbf(y * sg);
}

// silu_bf for N bf16 values at once, bit-identical to silu_bf on every bf16 input. For
// |y| < 8 the sigmoid comes from the hardware 2^x and reciprocal, rounded to bf16; a lane
// with any |y| >= 8 (or NaN) in its batch recomputes the whole batch on the exact path.
// The input is a bf16 value, so the domain is finite: that the fast value rounds to the
// same bf16 as d_sigmoidf(y) for every one of them is established by running all 65,536
// bf16 patterns through this function on the device against the exact path (the GPU test
// suite does, and through the prefill front end that uses it). The fast value is within
// 0.83 (5 + |y|) ulp of the exact one; no per-value midpoint test is made (one that fired
// would send about 40 % of the batches of a wave down the exact path for nothing).
template <int N>
__device__ __forceinline__ void silu_bf_batch(float (&y)[N]) {
  float sg[N];
  bool ok = true;
#pragma unroll
  for (int e = 0; e < N; ++e) {
    const float ex = __builtin_amdgcn_exp2f(-y[e] * 1.44269504088896341f);
    const float s = __builtin_amdgcn_rcpf(1.0f + ex);
    ok = ok & (__builtin_fabsf(y[e]) < 8.0f);
    sg[e] = rbf(s);
  }
  if (__builtin_expect(!ok, 0)) {
#pragma unroll
    for (int e = 0; e < N; ++e) sg[e] = rbf(d_sigmoidf(y[e]));
  }
#pragma unroll
  for (int e = 0; e < N; ++e) y[e] = rbf(y[e] * sg[e]);
}

// rbf(1 / sqrtf(d)) -- the l2norm's bf16 reciprocal square root of a bf16 value d
// (ops.cpp:27-30). The hardware v_rsq_f32 is within 1 ulp of 1 / sqrt(d) for normal d, so
// when its result lies more than 4 ulp from a bf16 rounding midpoint (0x8000 in the low 16
// bits) both round to the same bf16; otherwise (and for d below the normal range, which
// v_rsq_f32 flushes, or NaN) the correctly rounded path runs. v_sad_u16 sums the distances
// of both 16-bit halves, so the high half is cleared first: the test sees the low half only.
__device__ __forceinline__ float rsqrt_bf(float d) {
  const float f = __builtin_amdgcn_rsqf(d);
  if (d >= 1.17549435e-38f && __builtin_amdgcn_sad_u16(f_bits(f) & 0xFFFFu, 0x8000u, 0u) > 4u) return rbf(f);
  return rbf(1.0f / sqrtf(d));
}

// Sum over the 16 lanes of a DPP row; every lane receives the same total.
// quad_perm[1,0,3,2], quad_perm[2,3,0,1], row_half_mirror, row_mirror. When lane m of
// the row holds the partial sum of group m, this is the butterfly p[m] += p[m ^ s],
// s = 1, 2, 4, 8, bit for bit: after each step the lanes being combined hold equal
// values, so the mirrors pick the same operands the xor partners would.
__device__ __forceinline__ float row16_sum(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x141, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x140, 0xF, 0xF, true));
  return x;
}

// Gate math of cpp/src/model.cpp:608-612 for one (step, v-head).
__device__ __forceinline__ void d_gates(float a_logit, float b_logit, float A_log, float dt_bias,
                                        float& alpha, float& beta) {
  beta = d_sigmoidf(b_logit);
  const float t = a_logit + dt_bias;
  const float sp = d_softplusf(t);
  const float A = d_expf(A_log);
  const float m = A * sp;
  alpha = d_expf(-m);
}

}  // namespace gdn
