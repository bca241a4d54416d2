/*
 * gdn.h -- C ABI of the MI355X (gfx950) gated-delta recurrence library, libgdn.so.
 *
 * One Gated-DeltaNet layer's recurrent core, per the reference's per-layer call:
 *
 *   gates   beta  = sigmoid(b),  alpha = exp(-exp(A_log) * softplus(a + dt_bias))
 *   update  S_t   = alpha_t (I - beta_t k_t k_t^T) S_{t-1} + beta_t k_t v_t^T
 *   readout o_t   = S_t^T q_t            (taken after the update)
 *
 * with the fp32 state of each (batch, v-head) stored (Dv, Dk), Dk contiguous, and
 * Dk = Dv = 128. q and k carry num_k_heads heads; v-head h reads k-head
 * h / (num_v_heads / num_k_heads). An optional front end takes the 10240-channel
 * in_proj_qkv output instead of q,k,v and applies the causal depthwise conv (4 taps),
 * SiLU, l2norm (eps 1e-6) and the q scale 128^-0.5, with bf16 rounding after every op
 * as the reference's bf16 MLX ops do.
 *
 * Reference interfaces replaced (paths relative to the reference tree):
 *   gdn_run             delta::run            cpp/src/delta.hpp:66-68 (delta.cpp:137-173),
 *                       with the gate math of cpp/src/model.cpp:608-612 and, in the conv
 *                       front end, model.cpp:585-606 and DepthwiseConv model.cpp:385-395;
 *                       the call site it drops into is model.cpp:622-624.
 *   gdn_prefill_chunked chunked_delta         python/qwen35.py:365-431
 *   gdn_commit          DeltaCache::commit    cpp/src/model.cpp:439-457
 *   gdn_qlinear         Linear::operator()    cpp/src/model.cpp:356-372 (quantized), for
 *                       the layer's in_proj_* and, with GatedRMSNorm::operator()
 *                       (model.cpp:350-354) in front, its out_proj
 *   gdn_qlinear_workspace_size                 (sizes the workspace above; the
 *                       reference allocates inside MLX)
 *   gdn_available       delta::available      cpp/src/delta.hpp:51 (delta.cpp:133-135)
 *
 * Conventions
 *   - Every pointer is device memory owned by the caller; the library allocates no
 *     device memory on any entry point and keeps no per-call state. (gdn_qlinear_noalloc
 *     uses a fixed scratch array the library holds per device, see there.)
 *   - All tensors are dense, row-major, with a leading n_layers dimension: layer l of
 *     a tensor of per-layer size N starts at element l*N. n_layers > 1 runs that many
 *     independent layers in one launch (the layers of a model evaluated together, or
 *     a benchmark); n_layers = 1 is the reference's per-layer call.
 *   - Work is ordered on `stream` (a hipStream_t; NULL is the null stream). No entry
 *     point synchronises the device. Entry points are thread-safe.
 *   - Errors never cross the ABI as exceptions. A non-zero return names the class of
 *     error; gdn_last_error() returns this thread's message for the last failure.
 *     Shapes the kernels do not implement are errors, never a silent fallback.
 */
#ifndef GDN_H
#define GDN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN_ABI_VERSION 5
#define GDN_HEAD_DIM 128 /* Dk = Dv */
#define GDN_CONV_TAPS 4  /* conv kernel size; the conv state holds GDN_CONV_TAPS-1 rows */

typedef enum gdn_status {
  GDN_OK = 0,
  GDN_EINVAL = 1,      /* bad argument: null, shape, overlap, alignment, enum value */
  GDN_EUNSUPPORTED = 2, /* no gfx950 device */
  GDN_EDEVICE = 3      /* a HIP call failed; the message carries the HIP error */
} gdn_status;

typedef enum gdn_dtype { GDN_DTYPE_BF16 = 0, GDN_DTYPE_F32 = 1 } gdn_dtype;

typedef enum gdn_frontend {
  GDN_FRONTEND_QKV = 0, /* q, k, v given (already normalised, as delta::run takes them) */
  GDN_FRONTEND_CONV = 1 /* x = in_proj_qkv output; conv + SiLU + l2norm + q scale inside */
} gdn_frontend;

typedef enum gdn_gate_mode {
  GDN_GATES_RAW = 0,        /* a, b logits with A_log, dt_bias: the gate math runs inside */
  GDN_GATES_PRECOMPUTED = 1 /* alpha, beta given in fp32, as delta::run takes them */
} gdn_gate_mode;

/* Arithmetic of gdn_prefill_chunked (gdn_run computes in fp32 either way). */
typedef enum gdn_prefill_precision {
  GDN_PREFILL_ACCURATE = 0, /* the default, as the reference runs an fp32 kernel for every
                               window (cpp/src/model.cpp:619-624): the state products carry
                               fp32 accuracy -- V' formed as T' (V - e^G K S) with S, the
                               fp32 X = V - e^G K S and T' split into bf16 hi + lo, and V''
                               split for K^T V'' -- so the state the next window or decode
                               step starts from is within about 1e-5 (max|a-b|/max|b|;
                               measured 3e-6..8e-6) of the fp32 recurrence whatever the
                               gates */
  GDN_PREFILL_FAST = 1      /* the same V' with bf16 S, T' and V'' (X alone split), and M V'
                               on bf16 operands: the state ends about 2e-3 to 4e-3 from the
                               fp32 recurrence, the outputs within about 6e-3; about 0.85 of
                               the time at T = 4096 */
} gdn_prefill_precision;

typedef enum gdn_states_layout {
  GDN_STATES_BHT = 0, /* (B, Hv, T, Dv, Dk): the reference's S_all order (delta.cpp:88) */
  GDN_STATES_TBH = 1  /* (T, B, Hv, Dv, Dk): step t is one contiguous state, so a commit
                         can adopt it by pointer */
} gdn_states_layout;

/* Shapes below omit the leading n_layers dimension. C = 2*Hk*128 + Hv*128. */
typedef struct gdn_layer_args {
  int n_layers;    /* >= 1 */
  int batch;       /* B >= 0 */
  int seq_len;     /* T >= 0 steps per sequence (decode: 1) */
  int num_k_heads; /* Hk >= 1 */
  int num_v_heads; /* Hv, a multiple of Hk */

  int frontend; /* gdn_frontend */
  /* GDN_FRONTEND_QKV */
  const void* q; /* (B, T, Hk, 128), qkv_dtype */
  const void* k; /* (B, T, Hk, 128), qkv_dtype */
  const void* v; /* (B, T, Hv, 128), qkv_dtype */
  int qkv_dtype; /* gdn_dtype */
  /* GDN_FRONTEND_CONV */
  const void* x;             /* (B, T, C) bf16, channels [q | k | v] */
  const void* conv_weight;   /* (4, C) bf16, w[j, c] = conv1d.weight[c, 0, j] */
  const void* conv_state_in; /* (B, 3, C) bf16 pre-conv rows, or NULL for zeros */
  void* conv_state_out;      /* (B, 3, C) bf16 <- last 3 rows of [conv_state_in ; x], or
                                NULL; must not overlap conv_state_in */

  int gate_mode; /* gdn_gate_mode */
  /* GDN_GATES_RAW */
  const void* a;        /* (B, T, Hv) bf16 */
  const void* b;        /* (B, T, Hv) bf16 */
  const float* A_log;   /* (Hv) */
  const float* dt_bias; /* (Hv) */
  /* GDN_GATES_PRECOMPUTED */
  const float* alpha; /* (B, T, Hv) */
  const float* beta;  /* (B, T, Hv) */

  const float* state_in; /* (B, Hv, 128, 128), or NULL for a zero state; 16-byte aligned */
  float* state_out;      /* (B, Hv, 128, 128) final state, or NULL; may equal state_in
                            (in place), must not otherwise overlap it; 16-byte aligned */
  float* states;         /* per-step states (collect), or NULL; must not overlap state_in;
                            16-byte aligned. gdn_run only. */
  int states_layout;     /* gdn_states_layout */
  void* o;               /* (B, T, Hv, 128), o_dtype; never NULL */
  int o_dtype;           /* gdn_dtype */
  void* workspace;       /* gdn_prefill_chunked only: caller device memory of at least
                            gdn_prefill_workspace_size() bytes, 256-byte aligned */
  size_t workspace_bytes;
  void* stream;          /* hipStream_t */
  int prefill_precision; /* gdn_prefill_precision (0, GDN_PREFILL_ACCURATE, when zeroed):
                            gdn_prefill_chunked and gdn_prefill_workspace_size; gdn_run
                            accepts either value */
} gdn_layer_args;

/* Recurrent form for any T (decode T = 1; speculative verify with `states`). The
 * state is read once and written once per call; with `states` set, the state after
 * every step is written too and state_out may be NULL (record mode: the input state
 * is left untouched, model.cpp:630-633). */
int gdn_run(const gdn_layer_args* args);

/* Chunked form (chunk 64, WY/UT transform) for prefill; same arguments as gdn_run
 * except that `states` must be NULL, a workspace is required, o and x and conv_state_in
 * (conv front end) or q, k and v (qkv front end) must be 16-byte aligned, and the qkv
 * front end takes bf16 q, k, v only. Intra-chunk products run on bf16 MFMA with fp32 accumulation;
 * the state hand-off between chunks stays fp32; prefill_precision chooses how closely the
 * final state follows the fp32 recurrence (gdn_prefill_precision). The workspace contents
 * are scratch: they need no initialisation and are meaningless afterwards. */
int gdn_prefill_chunked(const gdn_layer_args* args);

/* gdn_prefill_chunked with a HIP event recorded before its first kernel and after each of
 * its three (the front end, the intra-chunk products, the chunk scan); it waits for the
 * last event and writes the kernels' durations in milliseconds to kernel_ms[0..2] (zeros
 * when nothing is launched). For measurement: unlike every other entry point it creates
 * events and waits for the stream. No counterpart in the reference (its callers are
 * benchmarks that report each kernel's share of the MFMA peak). */
int gdn_prefill_chunked_timed(const gdn_layer_args* args, float* kernel_ms);

/* Workspace bytes gdn_prefill_chunked needs for these arguments' batch, seq_len and head
 * counts (per chunk: Q, K, K^T, V, T' and the gate factors; the same for both front ends
 * and both precisions; prefill_precision is checked); the other fields are not read. */
int gdn_prefill_workspace_size(const gdn_layer_args* args, size_t* bytes);

typedef struct gdn_commit_args {
  int n_layers;    /* >= 1 */
  int batch;       /* B */
  int seq_len;     /* T of the recorded block */
  int num_v_heads; /* Hv */
  int conv_dim;    /* C; 0 skips the conv window */
  int n;           /* accepted prefix, 0 <= n <= T */
  const float* states;       /* as written by gdn_run */
  int states_layout;         /* gdn_states_layout */
  const float* state_prev;   /* (B, Hv, 128, 128): the state the block started from */
  float* state_dst;          /* (B, Hv, 128, 128) <- n == 0 ? state_prev : states[n-1];
                                may equal state_prev; with n_layers = 1 and the
                                GDN_STATES_TBH layout it may BE step n-1's block
                                (states + (n-1)*B*Hv*128*128): the pointer-swap commit,
                                which copies no state (only the conv window moves) */
  const void* conv_state_in; /* (B, 3, C) bf16 the block started from, or NULL (zeros) */
  const void* x;             /* (B, T, C) bf16, the block's conv input */
  void* conv_state_dst;      /* (B, 3, C) bf16 <- rows n..n+2 of [conv_state_in ; x]; may
                                equal conv_state_in */
  void* stream;              /* hipStream_t */
} gdn_commit_args;

/* DeltaCache::commit(n): accept the first n tokens of a recorded block. */
int gdn_commit(const gdn_commit_args* args);

/* ---- quantized linear: the DeltaNet layer's projections ----
 * y = x W^T with W in the reference's 4-bit affine layout, as Linear::operator() computes
 * it for quantized weights (cpp/src/model.cpp:356-372: mx::quantized_matmul, transpose
 * = true, group 64, bits 4; layout python/mlp_kernel.py:54-56): w (N, K/8) uint32 holds 8
 * values per word, value i in nibble i (low nibble first); element (n, k) = nibble *
 * scales[n, k/64] + biases[n, k/64]. The result is rounded to bf16 once. Up to
 * GDN_QLINEAR_MAX_SEGS matrices that read the same operand run in one launch: the
 * layer's in_proj_qkv, in_proj_z, in_proj_a and in_proj_b (model.cpp:587, 608-609, 626).
 * With norm_x set, the operand is the layer's GatedRMSNorm of the recurrence output
 * (model.cpp:350-354, 626-627), bf16(rmsnorm(norm_x) * norm_gamma * silu(norm_z)) over
 * each 128-value head, so norm + out_proj (model.cpp:641) is one call.
 * Up to GDN_QLINEAR_GEMV_ROWS operand rows (decode) the call needs no workspace; more
 * rows (verify blocks, batched decode, and prefill windows: the reference keeps
 * quantized_matmul below 512 rows and dequantizes and multiplies above, model.hpp:137,
 * model.cpp:358-362, in windows of 1024 tokens, session.hpp:136) run on MFMA with the same
 * exact arithmetic at every row count, up to GDN_QLINEAR_MAX_ROWS, and take a workspace of
 * gdn_qlinear_workspace_size() bytes for the operand in MFMA fragment order and its sums per
 * row and 64 values. */
#define GDN_QLINEAR_MAX_SEGS 4
#define GDN_QLINEAR_GEMV_ROWS 4
#define GDN_QLINEAR_MAX_ROWS 4096

typedef struct gdn_qlinear_seg {
  const void* w;      /* (N, K/8) uint32, 16-byte aligned */
  const void* scales; /* (N, K/64) bf16, 8-byte aligned */
  const void* biases; /* (N, K/64) bf16, 8-byte aligned */
  void* y;            /* (M, N) bf16; must not overlap any input */
  int n;              /* N >= 1 */
} gdn_qlinear_seg;

typedef struct gdn_qlinear_args {
  int n_layers; /* >= 1; layer l of every tensor starts at l times its per-layer size */
  int m;        /* rows of the operand (B * L), 1 .. GDN_QLINEAR_MAX_ROWS; up to
                   GDN_QLINEAR_GEMV_ROWS also m * k <= 30720 (else the MFMA path) */
  int k;        /* in features: 1024, 2048, 4096, 5120, 6144 or 8192 */
  const void* x; /* (M, K) bf16, 16-byte aligned; NULL when norm_x is set */
  const float* norm_x;     /* (M, K) fp32 (the recurrence output o), or NULL */
  const void* norm_z;      /* (M, K) bf16 gate z */
  const float* norm_gamma; /* (128) fp32 norm weight */
  float norm_eps;          /* >= 0 */
  int n_segs;   /* 1 .. GDN_QLINEAR_MAX_SEGS */
  gdn_qlinear_seg segs[GDN_QLINEAR_MAX_SEGS];
  void* workspace;        /* MFMA path only: device memory of at least
                             gdn_qlinear_workspace_size() bytes, 256-byte aligned; its
                             contents are scratch */
  size_t workspace_bytes;
  void* stream; /* hipStream_t */
} gdn_qlinear_args;

int gdn_qlinear(const gdn_qlinear_args* args);

/* Workspace bytes gdn_qlinear needs for these arguments' n_layers, m and k (0 on the
 * GEMV path); the other fields are not read. */
int gdn_qlinear_workspace_size(const gdn_qlinear_args* args, size_t* bytes);

/* gdn_qlinear without a workspace argument and without any allocation. No counterpart in
 * the reference (MLX allocates inside quantized_matmul): for callers that cannot allocate
 * device memory -- code under HIP graph capture, serving loops and harnesses that forbid
 * hipMalloc. Same arguments, kernels and results as gdn_qlinear, except that `workspace`
 * must be NULL and `workspace_bytes` 0: the MFMA path's operand and its group sums go to a
 * scratch array the library holds on each device (GDN_QLINEAR_NOALLOC_SCRATCH_BYTES, kept
 * until the process ends), so calls whose gdn_qlinear_workspace_size() exceeds that are
 * GDN_EINVAL (one layer of up to 512 rows at any k fits; 1024 rows fit for k up to 4096).
 * Every call on a device shares that device's scratch: calls that overlap in time on one
 * device (different streams or threads) race. */
#define GDN_QLINEAR_NOALLOC_SCRATCH_BYTES ((size_t)9 << 20)
int gdn_qlinear_noalloc(const gdn_qlinear_args* args);

/* 1 if the current HIP device is a gfx950 the kernels were built for, else 0. */
int gdn_available(void);

/* GDN_ABI_VERSION of the library. */
int gdn_abi_version(void);

/* This thread's message for the most recent failed call ("" if none). */
const char* gdn_last_error(void);

#ifdef __cplusplus
}
#endif
#endif /* GDN_H */
