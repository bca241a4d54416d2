// Launch parameters shared between the host entry points (gdn_api.cpp) and the
// kernels (*.hip). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gdn.h"

namespace gdn {

constexpr int kD = 128;     // Dk = Dv
constexpr int kTaps = 4;    // conv kernel
constexpr int kConvRows = kTaps - 1;

// Recurrent (decode / verify) launch. Every pointer already points at layer 0; the
// per-layer element counts below give the layer strides.
struct RecurrentParams {
  int n_layers, B, T, Hk, Hv, rep, C;
  int qkv_bf16;    // QKV front end: q,k,v dtype is bf16 (else fp32)
  int gate_raw;    // gates from a, b, A_log, dt_bias (else alpha, beta given)
  int o_bf16;      // o dtype is bf16 (else fp32)
  int states_tbh;  // states layout (T,B,Hv,Dv,Dk) (else (B,Hv,T,Dv,Dk))
  int remap;       // XCD-aware block order
  int nblocks;
  const void* q;
  const void* k;
  const void* v;
  const uint16_t* x;
  const uint16_t* conv_w;
  const uint16_t* conv_in;
  uint16_t* conv_out;
  const uint16_t* a;
  const uint16_t* b;
  const float* A_log;
  const float* dt_bias;
  const float* alpha;
  const float* beta;
  const float* state_in;
  float* state_out;
  float* states;
  void* o;
};

// frontend: 0 = q,k,v given, 1 = conv front end. collect: write per-step states.
hipError_t launch_recurrent(const RecurrentParams& p, int frontend, bool collect,
                            hipStream_t stream);

// Copies `n` floats (src may be null: zero fill) -- used for empty blocks.
hipError_t launch_copy_f32(float* dst, const float* src, int64_t n, hipStream_t stream);
hipError_t launch_copy_u16(uint16_t* dst, const uint16_t* src, int64_t n, hipStream_t stream);

struct CommitParams {
  int n_layers, B, T, Hv, C, n;
  int states_tbh;
  const float* states;
  const float* state_prev;
  float* state_dst;
  const uint16_t* conv_in;
  const uint16_t* x;
  uint16_t* conv_dst;
};
hipError_t launch_commit(const CommitParams& p, hipStream_t stream);

// Quantized linear (arguments validated by the caller).
bool qlinear_k_supported(int k);
// m rows of k on the GEMV path (no workspace); otherwise the MFMA path
bool qlinear_uses_gemv(int m, int k);
size_t qlinear_workspace_bytes(int n_layers, int m, int k);
hipError_t launch_qlinear(const gdn_qlinear_args& a, hipStream_t stream);
// Device address of this device's gdn_qlinear_noalloc scratch
// (GDN_QLINEAR_NOALLOC_SCRATCH_BYTES, 256-byte aligned), looked up once per device.
hipError_t qlinear_scratch(void** ptr);

}  // namespace gdn
