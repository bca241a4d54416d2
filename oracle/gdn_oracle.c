/*
 * CPU oracle for the gated-delta recurrence -- TEST INFRASTRUCTURE ONLY.
 *
 * A restatement of the reference's unfused MLX op sequence (file:line citations
 * on every function below and in gdn_oracle.h). Only tests/, the smoke check and
 * bench.py's CPU-baseline leg use it; the HIP product never does.
 *
 * Build flags matter: -ffp-contract=off keeps every multiply and add a separately
 * rounded fp32 operation, as MLX evaluates them (the reference builds with the same
 * flag, cpp/Makefile:90-99).
 */
#include "gdn_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define D GDNO_D

static int nthreads(int threads) {
#ifdef _OPENMP
  return threads > 0 ? threads : omp_get_max_threads();
#else
  (void)threads;
  return 1;
#endif
}

/* ------------------------------------------------------------------------- */
/* Generator: SplitMix64 (Steele, Lea, Flood 2014) seeds xoshiro256** (Blackman and
 * Vigna 2018); normals by the Box-Muller transform. */

uint64_t gdno_splitmix64_next(uint64_t* state) {
  uint64_t z = (*state += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

static inline uint64_t rotl64(uint64_t x, int k) { return (x << k) | (x >> (64 - k)); }

void gdno_xoshiro_seed(uint64_t s[4], uint64_t seed) {
  uint64_t sm = seed;
  for (int i = 0; i < 4; ++i) s[i] = gdno_splitmix64_next(&sm);
}

uint64_t gdno_xoshiro_next(uint64_t s[4]) {
  const uint64_t result = rotl64(s[1] * 5, 7) * 9;
  const uint64_t t = s[1] << 17;
  s[2] ^= s[0];
  s[3] ^= s[1];
  s[1] ^= s[2];
  s[0] ^= s[3];
  s[2] ^= t;
  s[3] = rotl64(s[3], 45);
  return result;
}

static inline double uniform01(uint64_t s[4]) {
  return (double)(gdno_xoshiro_next(s) >> 11) * 0x1.0p-53; /* [0, 1) */
}

void gdno_fill_normal(uint64_t seed, float mean, float std, float* out, int64_t n) {
  uint64_t s[4];
  gdno_xoshiro_seed(s, seed);
  const double two_pi = 6.283185307179586476925286766559;
  for (int64_t i = 0; i < n; i += 2) {
    const double u1 = 1.0 - uniform01(s); /* (0, 1] */
    const double u2 = uniform01(s);
    const double r = sqrt(-2.0 * log(u1));
    out[i] = (float)(mean + std * (r * cos(two_pi * u2)));
    if (i + 1 < n) out[i + 1] = (float)(mean + std * (r * sin(two_pi * u2)));
  }
}

void gdno_fill_uniform(uint64_t seed, float lo, float hi, float* out, int64_t n) {
  uint64_t s[4];
  gdno_xoshiro_seed(s, seed);
  for (int64_t i = 0; i < n; ++i) out[i] = (float)(lo + (hi - lo) * uniform01(s));
}

/* ------------------------------------------------------------------------- */
/* bf16 */

uint16_t gdno_f32_to_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float gdno_bf16_to_f32(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float x;
  memcpy(&x, &u, 4);
  return x;
}

static inline float rb(float x) { return gdno_bf16_to_f32(gdno_f32_to_bf16(x)); }

void gdno_round_bf16(const float* in, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = gdno_f32_to_bf16(in[i]);
}

void gdno_widen_bf16(const uint16_t* in, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = gdno_bf16_to_f32(in[i]);
}

/* ------------------------------------------------------------------------- */
/* fp32 elementary functions. MLX's own exp/log1p are not pinned at the ulp level
 * (no stored vectors exist); these are fixed, documented algorithms accurate to a
 * couple of ulp, checked against fp64 libm by the tests. */

static inline float f_from_bits(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}
static inline uint32_t bits_from_f(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}

/* exp: Cody-Waite reduction x = n ln2 + r, |r| <= ln2/2, then the degree-7 Taylor
 * polynomial of e^r by Horner with fused multiply-adds; 2^n applied in two halves
 * so that no intermediate overflows or underflows early. */
float gdno_expf(float x) {
  if (x != x) return x;
  if (x > 88.72283935546875f) return INFINITY;
  if (x < -103.97208404541015625f) return 0.0f;
  const float n = rintf(x * 1.44269502162933349609375f);
  float r = fmaf(-n, 0.693145751953125f, x);
  r = fmaf(-n, 1.428606765330187045e-06f, r);
  float p = 1.98412698412698412698e-4f;
  p = fmaf(p, r, 1.38888888888888888889e-3f);
  p = fmaf(p, r, 8.33333333333333333333e-3f);
  p = fmaf(p, r, 4.16666666666666666667e-2f);
  p = fmaf(p, r, 1.66666666666666666667e-1f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  const int ni = (int)n;
  const int n1 = ni / 2, n2 = ni - n1;
  p = p * f_from_bits((uint32_t)(n1 + 127) << 23);
  return p * f_from_bits((uint32_t)(n2 + 127) << 23);
}

/* log for positive normal x: x = m 2^e with m in [sqrt(1/2), sqrt(2)), f = m - 1
 * (exact), s = f/(2+f), log(1+f) = 2s + s R(s^2) with R(z) = 2z/3 + 2z^2/5 + 2z^3/7 +
 * 2z^4/9, evaluated as f - (f^2/2 - s (f^2/2 + R)) so the exact f carries the bulk. */
float gdno_logf(float x) {
  if (x != x || x < 0.0f) return NAN;
  if (x == 0.0f) return -INFINITY;
  if (x == INFINITY) return x;
  uint32_t u = bits_from_f(x);
  int e = (int)((u >> 23) & 0xffu) - 127;
  float m = f_from_bits((u & 0x007fffffu) | 0x3f800000u);
  if (m > 1.41421356237309504880f) {
    m = m * 0.5f;
    e += 1;
  }
  const float f = m - 1.0f;
  const float s = f / (2.0f + f);
  const float z = s * s;
  float R = 0.22222222222222222222f;             /* 2/9 */
  R = fmaf(R, z, 0.28571428571428571429f);       /* 2/7 */
  R = fmaf(R, z, 0.4f);                          /* 2/5 */
  R = fmaf(R, z, 0.66666666666666666667f);       /* 2/3 */
  R = R * z;
  const float hfsq = 0.5f * f * f;
  const float lm = f - (hfsq - s * (hfsq + R));
  const float ef = (float)e;
  return fmaf(ef, 0.693145751953125f, fmaf(ef, 1.428606765330187045e-06f, lm));
}

/* log1p with Goldberg's correction for the rounding of 1+x. */
float gdno_log1pf(float x) {
  const float w = 1.0f + x;
  if (w == 1.0f) return x;
  if (w == INFINITY) return w;
  return gdno_logf(w) * (x / (w - 1.0f));
}

/* sigmoid as MLX's unary op: 1 / (1 + exp(-x)). */
float gdno_sigmoidf(float x) {
  const float e = gdno_expf(-x);
  const float d = 1.0f + e;
  return 1.0f / d;
}

/* softplus = logaddexp(0, x) (cpp/src/ops.cpp:22-25):
 * max + log1p(exp(min - max)), returning max when min is -inf or max is +inf. */
float gdno_softplusf(float x) {
  const float mx = x > 0.0f ? x : 0.0f;
  const float mn = x > 0.0f ? 0.0f : x;
  if (x != x) return x;
  if (mn == -INFINITY || mx == INFINITY) return mx;
  return mx + gdno_log1pf(gdno_expf(mn - mx));
}

float gdno_rsqrtf(float x) { return 1.0f / sqrtf(x); }

/* ------------------------------------------------------------------------- */
/* gates: cpp/src/model.cpp:608-612 (python/qwen35.py:597-600). */

void gdno_gates(int64_t rows, int Hv, const uint16_t* a, const uint16_t* b,
                const float* A_log, const float* dt_bias, float* alpha, float* beta) {
  for (int64_t r = 0; r < rows; ++r) {
    for (int h = 0; h < Hv; ++h) {
      const int64_t i = r * Hv + h;
      beta[i] = gdno_sigmoidf(gdno_bf16_to_f32(b[i]));
      const float t = gdno_bf16_to_f32(a[i]) + dt_bias[h];
      const float sp = gdno_softplusf(t);
      const float A = gdno_expf(A_log[h]);
      const float m = A * sp;
      alpha[i] = gdno_expf(-m);
    }
  }
}

/* ------------------------------------------------------------------------- */
/* front end: DepthwiseConv (model.cpp:385-395), silu (ops.cpp:20),
 * l2norm (ops.cpp:27-30), q scale and split (model.cpp:588-602). Every op is a
 * bf16 MLX op: computed in fp32, rounded to bf16. */

float gdno_sum128_tree(const float* sq) {
  float p[64];
  for (int l = 0; l < 64; ++l) p[l] = sq[l] + sq[l + 64];
  for (int m = 1; m < 64; m <<= 1) {
    float nx[64];
    for (int l = 0; l < 64; ++l) nx[l] = p[l] + p[l ^ m];
    memcpy(p, nx, sizeof(p));
  }
  return p[0];
}

static void l2norm_bf16(const float* u, float scale_b, int apply_scale, uint16_t* out) {
  float sq[D];
  for (int d = 0; d < D; ++d) sq[d] = rb(u[d] * u[d]);
  const float s = rb(gdno_sum128_tree(sq));
  const float den = rb(s + rb(1e-6f));
  const float r = rb(gdno_rsqrtf(den));
  for (int d = 0; d < D; ++d) {
    float y = rb(u[d] * r);
    if (apply_scale) y = rb(y * scale_b);
    out[d] = gdno_f32_to_bf16(y);
  }
}

void gdno_conv_frontend(int B, int L, int Hk, int Hv, const uint16_t* x,
                        const uint16_t* conv_state, const uint16_t* w, uint16_t* q,
                        uint16_t* k, uint16_t* v, uint16_t* xp) {
  const int C = 2 * Hk * D + Hv * D;
  const int KC = GDNO_KCONV;
  const float scale_b = rb(1.0f / sqrtf((float)D));
  float* u = (float*)malloc(sizeof(float) * (size_t)C);
  for (int b = 0; b < B; ++b) {
    for (int t = 0; t < L; ++t) {
      /* conv output for every channel at step t; xp row r is conv_state[r] for r<3 */
      for (int c = 0; c < C; ++c) {
        float y = 0.0f;
        for (int j = 0; j < KC; ++j) {
          const int r = t + j;
          float xv;
          if (r < KC - 1) {
            xv = conv_state ? gdno_bf16_to_f32(conv_state[((int64_t)b * (KC - 1) + r) * C + c]) : 0.0f;
          } else {
            xv = gdno_bf16_to_f32(x[((int64_t)b * L + (r - (KC - 1))) * C + c]);
          }
          const float prod = rb(xv * gdno_bf16_to_f32(w[(int64_t)j * C + c]));
          y = (j == 0) ? prod : rb(y + prod);
        }
        const float sg = rb(gdno_sigmoidf(y));
        u[c] = rb(y * sg);
      }
      const int64_t row = (int64_t)b * L + t;
      for (int g = 0; g < Hk; ++g) {
        l2norm_bf16(u + g * D, scale_b, 1, q + (row * Hk + g) * D);
        l2norm_bf16(u + Hk * D + g * D, scale_b, 0, k + (row * Hk + g) * D);
      }
      for (int i = 0; i < Hv * D; ++i) v[row * Hv * D + i] = gdno_f32_to_bf16(u[2 * Hk * D + i]);
    }
    if (xp) {
      for (int r = 0; r < L + KC - 1; ++r) {
        for (int c = 0; c < C; ++c) {
          uint16_t val;
          if (r < KC - 1) {
            val = conv_state ? conv_state[((int64_t)b * (KC - 1) + r) * C + c] : 0;
          } else {
            val = x[((int64_t)b * L + (r - (KC - 1))) * C + c];
          }
          xp[((int64_t)b * (L + KC - 1) + r) * C + c] = val;
        }
      }
    }
  }
  free(u);
}

/* ------------------------------------------------------------------------- */
/* recurrence: cpp/src/delta.cpp:185-200, per step on (B,H,Dv,Dk):
 *   kS = sum(k_t * S, -1);  S = a_t*(S - b_t*(kS*k_t)) + b_t*(v_t*k_t);  o = sum(q_t * S, -1)
 * Reductions over Dk run in index order. */

static void recurrent_fused(int B, int L, int Hk, int Hv, const float* q, const float* k,
                            const float* v, const float* alpha, const float* beta,
                            float* S, float* o, float* states, int nt) {
  const int rep = Hv / Hk;
#pragma omp parallel for collapse(2) schedule(static) num_threads(nt)
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < Hv; ++h) {
      float* Sh = S + ((int64_t)b * Hv + h) * D * D;
      for (int t = 0; t < L; ++t) {
        const int64_t row = (int64_t)b * L + t;
        const float* kt = k + (row * Hk + h / rep) * D;
        const float* qt = q + (row * Hk + h / rep) * D;
        const float* vt = v + (row * Hv + h) * D;
        const float a = alpha[row * Hv + h], bb = beta[row * Hv + h];
        for (int r = 0; r < D; ++r) {
          float* s = Sh + (int64_t)r * D;
          float kS = 0.0f;
          for (int d = 0; d < D; ++d) kS += kt[d] * s[d];
          float ov = 0.0f;
          for (int d = 0; d < D; ++d) {
            const float p2 = kS * kt[d];
            const float p3 = bb * p2;
            const float p4 = s[d] - p3;
            const float p5 = a * p4;
            const float p6 = vt[r] * kt[d];
            const float p7 = bb * p6;
            s[d] = p5 + p7;
          }
          for (int d = 0; d < D; ++d) ov += qt[d] * s[d];
          o[(row * Hv + h) * D + r] = ov;
        }
        if (states) {
          memcpy(states + ((((int64_t)b * Hv + h) * L + t) * D) * D, Sh, sizeof(float) * D * D);
        }
      }
    }
  }
}

/* One full pass per MLX op over materialised state-sized temporaries -- the
 * structure of the unfused op graph, used as the timed CPU baseline. */
static void recurrent_materialized(int B, int L, int Hk, int Hv, const float* q,
                                   const float* k, const float* v, const float* alpha,
                                   const float* beta, float* S, float* o, float* states,
                                   int nt) {
  const int rep = Hv / Hk;
  const int64_t nrow = (int64_t)B * Hv * D; /* (b, h, r) rows */
  const int64_t n = nrow * D;
  float* P1 = (float*)malloc(sizeof(float) * n);
  float* P2 = (float*)malloc(sizeof(float) * n);
  float* kS = (float*)malloc(sizeof(float) * nrow);
  for (int t = 0; t < L; ++t) {
#define KT(i) (k[(((int64_t)((i) / ((int64_t)Hv * D * D)) * L + t) * Hk + (((i) / ((int64_t)D * D)) % Hv) / rep) * D + (i) % D])
#define QT(i) (q[(((int64_t)((i) / ((int64_t)Hv * D * D)) * L + t) * Hk + (((i) / ((int64_t)D * D)) % Hv) / rep) * D + (i) % D])
#define AT(i) (alpha[((int64_t)((i) / ((int64_t)Hv * D * D)) * L + t) * Hv + ((i) / ((int64_t)D * D)) % Hv])
#define BT(i) (beta[((int64_t)((i) / ((int64_t)Hv * D * D)) * L + t) * Hv + ((i) / ((int64_t)D * D)) % Hv])
#define VT(i) (v[(((int64_t)((i) / ((int64_t)Hv * D * D)) * L + t) * Hv + ((i) / ((int64_t)D * D)) % Hv) * D + ((i) / D) % D])
    /* P1 = k_t * S */
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < n; ++i) P1[i] = KT(i) * S[i];
    /* kS = sum(P1, -1) */
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t r = 0; r < nrow; ++r) {
      float acc = 0.0f;
      for (int d = 0; d < D; ++d) acc += P1[r * D + d];
      kS[r] = acc;
    }
    /* P2 = kS * k_t */
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < n; ++i) P2[i] = kS[i / D] * KT(i);
    /* P1 = b_t * P2 */
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < n; ++i) P1[i] = BT(i) * P2[i];
    /* P2 = S - P1 */
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < n; ++i) P2[i] = S[i] - P1[i];
    /* S = a_t * P2 (the old S is dead after this point) */
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < n; ++i) S[i] = AT(i) * P2[i];
    /* P1 = v_t * k_t */
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < n; ++i) P1[i] = VT(i) * KT(i);
    /* P2 = b_t * P1 */
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < n; ++i) P2[i] = BT(i) * P1[i];
    /* S = S + P2 */
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < n; ++i) S[i] = S[i] + P2[i];
    /* P1 = q_t * S;  o = sum(P1, -1) */
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t i = 0; i < n; ++i) P1[i] = QT(i) * S[i];
#pragma omp parallel for schedule(static) num_threads(nt)
    for (int64_t r = 0; r < nrow; ++r) {
      float acc = 0.0f;
      for (int d = 0; d < D; ++d) acc += P1[r * D + d];
      const int64_t b = r / ((int64_t)Hv * D), h = (r / D) % Hv, rr = r % D;
      o[(((int64_t)b * L + t) * Hv + h) * D + rr] = acc;
    }
    if (states) {
#pragma omp parallel for schedule(static) num_threads(nt)
      for (int64_t bh = 0; bh < (int64_t)B * Hv; ++bh) {
        memcpy(states + ((bh * L + t) * D) * D, S + bh * D * D, sizeof(float) * D * D);
      }
    }
#undef KT
#undef QT
#undef AT
#undef BT
#undef VT
  }
  free(P1);
  free(P2);
  free(kS);
}

void gdno_recurrent_f32(int B, int L, int Hk, int Hv, const float* q, const float* k,
                        const float* v, const float* alpha, const float* beta,
                        const float* S_in, float* S_out, float* o, float* states,
                        int materialize, int threads) {
  const int64_t ns = (int64_t)B * Hv * D * D;
  if (S_in) {
    if (S_in != S_out) memcpy(S_out, S_in, sizeof(float) * ns);
  } else {
    memset(S_out, 0, sizeof(float) * ns);
  }
  const int nt = nthreads(threads);
  if (materialize) {
    recurrent_materialized(B, L, Hk, Hv, q, k, v, alpha, beta, S_out, o, states, nt);
  } else {
    recurrent_fused(B, L, Hk, Hv, q, k, v, alpha, beta, S_out, o, states, nt);
  }
}

void gdno_recurrent_f64(int B, int L, int Hk, int Hv, const float* q, const float* k,
                        const float* v, const float* alpha, const float* beta,
                        const float* S_in, double* S, double* o, int threads) {
  const int rep = Hv / Hk;
  const int nt = nthreads(threads);
  const int64_t ns = (int64_t)B * Hv * D * D;
  for (int64_t i = 0; i < ns; ++i) S[i] = S_in ? (double)S_in[i] : 0.0;
#pragma omp parallel for collapse(2) schedule(static) num_threads(nt)
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < Hv; ++h) {
      double* Sh = S + ((int64_t)b * Hv + h) * D * D;
      for (int t = 0; t < L; ++t) {
        const int64_t row = (int64_t)b * L + t;
        const float* kt = k + (row * Hk + h / rep) * D;
        const float* qt = q + (row * Hk + h / rep) * D;
        const float* vt = v + (row * Hv + h) * D;
        const double a = alpha[row * Hv + h], bb = beta[row * Hv + h];
        for (int r = 0; r < D; ++r) {
          double* s = Sh + (int64_t)r * D;
          double kS = 0.0, ov = 0.0;
          for (int d = 0; d < D; ++d) kS += (double)kt[d] * s[d];
          for (int d = 0; d < D; ++d) {
            s[d] = a * (s[d] - bb * kS * (double)kt[d]) + bb * (double)vt[r] * (double)kt[d];
            ov += (double)qt[d] * s[d];
          }
          o[(row * Hv + h) * D + r] = ov;
        }
      }
    }
  }
}

/* ------------------------------------------------------------------------- */
/* chunked form: python/qwen35.py:365-431 with _invert_unit_lower (350-362).
 * Internally S is (Dk, Dv) per head, as in the reference (qwen35.py:419-422). */

void gdno_chunked_f32(int B, int L, int Hk, int Hv, int C, const float* q, const float* k,
                      const float* v, const float* alpha, const float* beta,
                      const float* S_in, float* S_out, float* o, int threads) {
  const int rep = Hv / Hk;
  const int nt = nthreads(threads);
  const int nC = (L + C - 1) / C;
#pragma omp parallel for collapse(2) schedule(dynamic) num_threads(nt)
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < Hv; ++h) {
      float* St = (float*)malloc(sizeof(float) * D * D); /* (Dk, Dv) */
      float* qc = (float*)malloc(sizeof(float) * C * D);
      float* kc = (float*)malloc(sizeof(float) * C * D);
      float* vc = (float*)malloc(sizeof(float) * C * D);
      float* g = (float*)malloc(sizeof(float) * C);
      float* bt = (float*)malloc(sizeof(float) * C);
      float* lcg = (float*)malloc(sizeof(float) * C);
      float* cumg = (float*)malloc(sizeof(float) * C);
      float* dr = (float*)malloc(sizeof(float) * C * C);
      float* Am = (float*)malloc(sizeof(float) * C * C);
      float* Ti = (float*)malloc(sizeof(float) * C * C);
      float* M = (float*)malloc(sizeof(float) * C * C);
      float* tmp = (float*)malloc(sizeof(float) * C * D);
      float* U0 = (float*)malloc(sizeof(float) * C * D);
      float* Kt = (float*)malloc(sizeof(float) * C * D);
      float* Qeff = (float*)malloc(sizeof(float) * C * D);
      float* MU0 = (float*)malloc(sizeof(float) * C * D);
      float* Uc = (float*)malloc(sizeof(float) * C * D);
      float* ratio = (float*)malloc(sizeof(float) * C);

      const float* Sh = S_in ? S_in + ((int64_t)b * Hv + h) * D * D : NULL;
      for (int i = 0; i < D; ++i)
        for (int j = 0; j < D; ++j) St[i * D + j] = Sh ? Sh[(int64_t)j * D + i] : 0.0f;

      for (int c = 0; c < nC; ++c) {
        /* gather the chunk; padded steps have q=k=v=0, alpha=1, beta=0 (381-388) */
        for (int i = 0; i < C; ++i) {
          const int t = c * C + i;
          if (t < L) {
            const int64_t row = (int64_t)b * L + t;
            memcpy(qc + i * D, q + (row * Hk + h / rep) * D, sizeof(float) * D);
            memcpy(kc + i * D, k + (row * Hk + h / rep) * D, sizeof(float) * D);
            memcpy(vc + i * D, v + (row * Hv + h) * D, sizeof(float) * D);
            g[i] = alpha[row * Hv + h];
            bt[i] = beta[row * Hv + h];
          } else {
            memset(qc + i * D, 0, sizeof(float) * D);
            memset(kc + i * D, 0, sizeof(float) * D);
            memset(vc + i * D, 0, sizeof(float) * D);
            g[i] = 1.0f;
            bt[i] = 0.0f;
          }
        }
        /* lcg = cumsum(log(clip(g, 1e-6, 1))); cumg = exp(lcg)  (400-401) */
        float acc = 0.0f;
        for (int i = 0; i < C; ++i) {
          float gi = g[i] < 1e-6f ? 1e-6f : (g[i] > 1.0f ? 1.0f : g[i]);
          acc = acc + logf(gi);
          lcg[i] = acc;
          cumg[i] = expf(lcg[i]);
        }
        /* dr[i,j] = exp(lcg_i - lcg_j) for j <= i, exp(-1e30) = 0 above (406) */
        for (int i = 0; i < C; ++i)
          for (int j = 0; j < C; ++j) dr[i * C + j] = j <= i ? expf(lcg[i] - lcg[j]) : 0.0f;
        /* A = bt_i * dr * (k k^T) * strict_lower (408) */
        for (int i = 0; i < C; ++i) {
          for (int j = 0; j < C; ++j) {
            float kk = 0.0f;
            for (int d = 0; d < D; ++d) kk += kc[i * D + d] * kc[j * D + d];
            const float sl = j < i ? 1.0f : 0.0f;
            Am[i * C + j] = ((bt[i] * dr[i * C + j]) * kk) * sl;
          }
        }
        /* Tinv = (I + A)^-1 by forward substitution over rows (358-362) */
        for (int i = 0; i < C; ++i) {
          for (int j = 0; j < C; ++j) {
            float acc2 = 0.0f;
            for (int m = 0; m < i; ++m) acc2 += Am[i * C + m] * Ti[m * C + j];
            Ti[i * C + j] = (i == j ? 1.0f : 0.0f) - acc2;
          }
        }
        /* U0 = Tinv (bt v);  Kt = Tinv ((bt cumg) k)   (411-412) */
        for (int i = 0; i < C; ++i)
          for (int d = 0; d < D; ++d) tmp[i * D + d] = bt[i] * vc[i * D + d];
        for (int i = 0; i < C; ++i)
          for (int d = 0; d < D; ++d) {
            float a2 = 0.0f;
            for (int m = 0; m < C; ++m) a2 += Ti[i * C + m] * tmp[m * D + d];
            U0[i * D + d] = a2;
          }
        for (int i = 0; i < C; ++i) {
          const float f = bt[i] * cumg[i];
          for (int d = 0; d < D; ++d) tmp[i * D + d] = f * kc[i * D + d];
        }
        for (int i = 0; i < C; ++i)
          for (int d = 0; d < D; ++d) {
            float a2 = 0.0f;
            for (int m = 0; m < C; ++m) a2 += Ti[i * C + m] * tmp[m * D + d];
            Kt[i * D + d] = a2;
          }
        /* M = dr * (q k^T) * lower; Qeff = cumg q - M Kt; MU0 = M U0 (413-415) */
        for (int i = 0; i < C; ++i)
          for (int j = 0; j < C; ++j) {
            float qk = 0.0f;
            for (int d = 0; d < D; ++d) qk += qc[i * D + d] * kc[j * D + d];
            const float lo = j <= i ? 1.0f : 0.0f;
            M[i * C + j] = (dr[i * C + j] * qk) * lo;
          }
        for (int i = 0; i < C; ++i)
          for (int d = 0; d < D; ++d) {
            float mk = 0.0f, mu = 0.0f;
            for (int m = 0; m < C; ++m) {
              mk += M[i * C + m] * Kt[m * D + d];
              mu += M[i * C + m] * U0[m * D + d];
            }
            Qeff[i * D + d] = cumg[i] * qc[i * D + d] - mk;
            MU0[i * D + d] = mu;
          }
        const float cumg_last = cumg[C - 1];
        for (int i = 0; i < C; ++i) ratio[i] = expf(lcg[C - 1] - lcg[i]); /* (417) */
        /* y = MU0 + Qeff S; Uc = U0 - Kt S; S = cumg_last S + k^T (ratio Uc) (424-429) */
        for (int i = 0; i < C; ++i) {
          const int t = c * C + i;
          for (int e = 0; e < D; ++e) {
            float qs = 0.0f, ks = 0.0f;
            for (int d = 0; d < D; ++d) {
              qs += Qeff[i * D + d] * St[d * D + e];
              ks += Kt[i * D + d] * St[d * D + e];
            }
            if (t < L) o[(((int64_t)b * L + t) * Hv + h) * D + e] = MU0[i * D + e] + qs;
            Uc[i * D + e] = ratio[i] * (U0[i * D + e] - ks);
          }
        }
        for (int d = 0; d < D; ++d)
          for (int e = 0; e < D; ++e) {
            float ku = 0.0f;
            for (int i = 0; i < C; ++i) ku += kc[i * D + d] * Uc[i * D + e];
            St[d * D + e] = cumg_last * St[d * D + e] + ku;
          }
      }
      float* So = S_out + ((int64_t)b * Hv + h) * D * D;
      for (int i = 0; i < D; ++i)
        for (int j = 0; j < D; ++j) So[(int64_t)j * D + i] = St[i * D + j];
      free(St); free(qc); free(kc); free(vc); free(g); free(bt); free(lcg); free(cumg);
      free(dr); free(Am); free(Ti); free(M); free(tmp); free(U0); free(Kt); free(Qeff);
      free(MU0); free(Uc); free(ratio);
    }
  }
}

/* ------------------------------------------------------------------------- */
/* DeltaCache::commit, cpp/src/model.cpp:439-457. */

int gdno_commit(int B, int T, int Hv, int C, int n, const float* states,
                const float* S_prev, const uint16_t* xp, float* S_dst, uint16_t* conv_dst) {
  if (n < 0 || n > T) return -1;
  const int KC = GDNO_KCONV;
  for (int b = 0; b < B; ++b) {
    for (int h = 0; h < Hv; ++h) {
      const float* src = (n == 0) ? S_prev + ((int64_t)b * Hv + h) * D * D
                                  : states + ((((int64_t)b * Hv + h) * T + (n - 1)) * D) * D;
      memmove(S_dst + ((int64_t)b * Hv + h) * D * D, src, sizeof(float) * D * D);
    }
    for (int r = 0; r < KC - 1; ++r) {
      memcpy(conv_dst + ((int64_t)b * (KC - 1) + r) * C,
             xp + ((int64_t)b * (T + KC - 1) + n + r) * C, sizeof(uint16_t) * C);
    }
  }
  return 0;
}

/* ------------------------------------------------------------------------- */
/* Quantized linear, cpp/src/model.cpp:356-372 (mx::quantized_matmul, transpose = true,
 * group 64, 4 bits): 8 values per uint32, value i in nibble i, low nibble first
 * (python/mlp_kernel.py:54-56), element = nibble * scale + bias. */

void gdno_qlinear_f64(int M, int N, int K, const uint16_t* x, const uint32_t* w,
                      const uint16_t* scales, const uint16_t* biases, double* y) {
  const int G = K / 64;
  for (int n = 0; n < N; ++n) {
    for (int m = 0; m < M; ++m) {
      double acc = 0.0;
      for (int k = 0; k < K; ++k) {
        const uint32_t word = w[(int64_t)n * (K / 8) + k / 8];
        const double nib = (double)((word >> (4 * (k % 8))) & 0xFu);
        const double s = gdno_bf16_to_f32(scales[(int64_t)n * G + k / 64]);
        const double bb = gdno_bf16_to_f32(biases[(int64_t)n * G + k / 64]);
        acc += (double)gdno_bf16_to_f32(x[(int64_t)m * K + k]) * (nib * s + bb);
      }
      y[(int64_t)m * N + n] = acc;
    }
  }
}

/* ------------------------------------------------------------------------- */
/* GatedRMSNorm, cpp/src/model.cpp:350-354: fast::rms_norm in fp32 (x * rsqrt(mean(x^2) +
 * eps) * w), then times silu(fp32(z)), rounded to the activation dtype (bf16). */

void gdno_gated_rmsnorm(int64_t rows, int dim, const float* o, const uint16_t* z,
                        const float* gamma, float eps, uint16_t* out) {
  for (int64_t r = 0; r < rows; ++r) {
    const float* x = o + r * dim;
    float ss = 0.0f;
    for (int i = 0; i < dim; ++i) ss += x[i] * x[i];
    const float rs = 1.0f / sqrtf(ss / (float)dim + eps);
    for (int i = 0; i < dim; ++i) {
      const float h = x[i] * rs * gamma[i];
      const float zf = gdno_bf16_to_f32(z[r * dim + i]);
      const float g = zf * gdno_sigmoidf(zf);
      out[r * dim + i] = gdno_f32_to_bf16(h * g);
    }
  }
}
