/*
 * CPU oracle for the gated-delta recurrence -- TEST INFRASTRUCTURE ONLY.
 *
 * This library restates, op for op, the reference's unfused MLX sequence for the
 * Gated-DeltaNet path. It is what the HIP kernels are compared with in the tests,
 * and the CPU baseline that bench.py times next to them. Nothing in the product
 * (the HIP library and its host code) may link, load or call it.
 *
 * Reference files it follows (paths relative to the reference tree):
 *   cpp/src/model.cpp:582-642   GatedDeltaNet::operator()  (front end, gates, record/advance)
 *   cpp/src/model.cpp:385-395   DepthwiseConv::operator()  (tap order, padded input)
 *   cpp/src/model.cpp:439-457   DeltaCache::commit
 *   cpp/src/ops.cpp:20-30       silu, softplus = logaddexp(0,x), l2norm (eps 1e-6, no 1/sqrt(d))
 *   cpp/src/delta.cpp:175-204   delta::run_reference       (per-step op order, collect layout)
 *   python/qwen35.py:350-431    _invert_unit_lower, chunked_delta
 *   python/qwen35.py:434-475    _delta_step, sequential_delta
 *   cpp/src/model.cpp:356-372   Linear::operator(), quantized branch (mx::quantized_matmul,
 *                               4-bit affine, group 64; layout python/mlp_kernel.py:54-56)
 *   cpp/src/model.cpp:350-354   GatedRMSNorm::operator() (normalise, then gate)
 *
 * Conventions: bf16 tensors are passed as uint16 bit patterns; fp32 state is
 * (B, Hv, Dv, Dk) with Dk contiguous; q,k carry Hk heads and v-head h reads k-head
 * h / (Hv/Hk) (repeat-interleave, model.cpp:603-605). Dk = Dv = 128.
 */
#ifndef GDN_ORACLE_H
#define GDN_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDNO_D 128   /* Dk = Dv */
#define GDNO_KCONV 4 /* conv taps */

/* ---- seeded generator: SplitMix64 seeding xoshiro256**, Box-Muller normals ---- */
uint64_t gdno_splitmix64_next(uint64_t* state);
void gdno_xoshiro_seed(uint64_t s[4], uint64_t seed);
uint64_t gdno_xoshiro_next(uint64_t s[4]);
void gdno_fill_normal(uint64_t seed, float mean, float std, float* out, int64_t n);
void gdno_fill_uniform(uint64_t seed, float lo, float hi, float* out, int64_t n);

/* ---- bf16 (round to nearest even) ---- */
uint16_t gdno_f32_to_bf16(float x);
float gdno_bf16_to_f32(uint16_t h);
void gdno_round_bf16(const float* in, uint16_t* out, int64_t n);
void gdno_widen_bf16(const uint16_t* in, float* out, int64_t n);

/* ---- fp32 elementary functions used by the op sequence ---- */
float gdno_expf(float x);
float gdno_logf(float x);
float gdno_log1pf(float x);
float gdno_sigmoidf(float x);
float gdno_softplusf(float x); /* logaddexp(0, x) */
float gdno_rsqrtf(float x);

/* ---- gates, model.cpp:608-612 ----
 * beta  = sigmoid(f32(b));  alpha = exp(-(exp(A_log) * softplus(f32(a) + dt_bias)))
 * a, b: (rows, Hv) bf16; A_log, dt_bias: (Hv,) fp32; alpha, beta: (rows, Hv) fp32 */
void gdno_gates(int64_t rows, int Hv, const uint16_t* a, const uint16_t* b,
                const float* A_log, const float* dt_bias, float* alpha, float* beta);

/* ---- front end, model.cpp:585-606 and 385-395 ----
 * x: (B, L, C) bf16 with C = 2*Hk*128 + Hv*128, channel split [q | k | v];
 * conv_state: (B, 3, C) bf16 or NULL (zeros); w: (4, C) bf16 (w[j,c] = conv1d.weight[c,0,j]).
 * Outputs (bf16): q, k (B, L, Hk, 128) -- silu, l2norm, q *= bf16(128^-0.5);
 * v (B, L, Hv, 128) -- silu only; xp (B, L+3, C) = [conv_state ; x] or NULL. */
void gdno_conv_frontend(int B, int L, int Hk, int Hv, const uint16_t* x,
                        const uint16_t* conv_state, const uint16_t* w, uint16_t* q,
                        uint16_t* k, uint16_t* v, uint16_t* xp);

/* The l2norm sum order this oracle fixes for the (unpinned) MLX bf16 reduction:
 * p[l] = sq[l] + sq[l+64] for l < 64, then six butterfly levels p[l] += p[l^m]. */
float gdno_sum128_tree(const float* sq);

/* ---- recurrence, delta.cpp:175-204 (run_reference) ----
 * q, k: (B, L, Hk, 128) fp32; v: (B, L, Hv, 128) fp32; alpha, beta: (B, L, Hv) fp32;
 * S_in: (B, Hv, 128, 128) or NULL (zeros); S_out: (B, Hv, 128, 128) (may equal S_in);
 * o: (B, L, Hv, 128); states: (B, Hv, L, 128, 128) or NULL.
 * materialize=1 runs one full pass per MLX op over state-sized temporaries (the
 * CPU baseline); materialize=0 runs the same per-element op sequence in one loop
 * (bit-identical, faster). threads<=0 uses every core. */
void gdno_recurrent_f32(int B, int L, int Hk, int Hv, const float* q, const float* k,
                        const float* v, const float* alpha, const float* beta,
                        const float* S_in, float* S_out, float* o, float* states,
                        int materialize, int threads);

/* Same recurrence in fp64 on the same fp32 inputs: the truth the fp32 paths are
 * measured against. S_out and o are fp64. */
void gdno_recurrent_f64(int B, int L, int Hk, int Hv, const float* q, const float* k,
                        const float* v, const float* alpha, const float* beta,
                        const float* S_in, double* S_out, double* o, int threads);

/* ---- chunked form, qwen35.py:350-431 (chunked_delta), fp32, chunk C ----
 * Same argument layouts as gdno_recurrent_f32 (no collect). */
void gdno_chunked_f32(int B, int L, int Hk, int Hv, int C, const float* q, const float* k,
                      const float* v, const float* alpha, const float* beta,
                      const float* S_in, float* S_out, float* o, int threads);

/* ---- DeltaCache::commit(n), model.cpp:439-457 ----
 * states: (B, Hv, T, 128, 128); S_prev: (B, Hv, 128, 128); xp: (B, T+3, C) bf16.
 * S_dst <- n == 0 ? S_prev : states[:, :, n-1];  conv_dst (B, 3, C) <- xp[:, n:n+3].
 * Returns 0, or -1 when n is outside [0, T] (the reference throws). */
int gdno_commit(int B, int T, int Hv, int C, int n, const float* states,
                const float* S_prev, const uint16_t* xp, float* S_dst, uint16_t* conv_dst);

/* ---- quantized linear, model.cpp:356-372 (mx::quantized_matmul, transpose = true) ----
 * x (M, K) bf16; w (N, K/8) uint32, value i of a word in nibble i (low nibble first);
 * scales, biases (N, K/64) bf16; element (n, k) = nibble * scale[n, k/64] + bias[n, k/64].
 * y (M, N) = x W^T accumulated in fp64 (the reference rounds its result to bf16). */
void gdno_qlinear_f64(int M, int N, int K, const uint16_t* x, const uint32_t* w,
                      const uint16_t* scales, const uint16_t* biases, double* y);

/* ---- GatedRMSNorm, model.cpp:350-354 ----
 * rows of D fp32 values o, bf16 gate z, fp32 gamma (D): h = o * rsqrt(mean(o^2) + eps) * gamma
 * in fp32 (mx::fast::rms_norm), out = bf16(h * silu(fp32(z))), silu(z) = z * sigmoid(z). */
void gdno_gated_rmsnorm(int64_t rows, int dim, const float* o, const uint16_t* z,
                        const float* gamma, float eps, uint16_t* out);

#ifdef __cplusplus
}
#endif
#endif
