// Launch parameters shared between the host entry points (gdn_api.cpp) and the
// kernels (*.hip). Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/gdn.h"

namespace gdn {

constexpr int kD = 128;     // Dk = Dv
constexpr int kTaps = 4;    // conv kernel
constexpr int kConvRows = kTaps - 1;

// Recurrent (decode / verify) launch. Every pointer already points at layer 0; the
// per-layer element counts below give the layer strides.
struct RecurrentParams {
  // Everything the T = 1 kernels read comes first and fits in 128 bytes, two 64-byte lines
  // of the kernarg segment: a single-layer decode is a chain of dependent latencies, and
  // every further line a workgroup reads costs a scalar-cache miss before its first load
  // can go out (with the reciprocals below, one layer at B = 1 went from 4.10 to 3.72 us
  // with q, k, v given and from 4.30 to 4.11 us with the conv front end).
  int B, Hk, Hv, rep;
  uint32_t rc_grp8, rc_hv, rc_b, rc_rep;  // ceil(2^32 / d) for the block map's divisors (0 for d = 1)
  unsigned qkv_bf16 : 1;    // QKV front end: q,k,v dtype is bf16 (else fp32)
  unsigned gate_raw : 1;    // gates from a, b, A_log, dt_bias (else alpha, beta given)
  unsigned o_bf16 : 1;      // o dtype is bf16 (else fp32)
  unsigned states_tbh : 1;  // states layout (T,B,Hv,Dv,Dk) (else (B,Hv,T,Dv,Dk))
  unsigned order : 2;       // block order: 0 dispatch, 1 contiguous split per XCD, 2 k-head groups interleaved
  unsigned fastdiv : 1;     // the reciprocals give every quotient of the block map exactly
  int C;                    // conv channels
  union { const void* q; const uint16_t* x; };       // q (QKV front end) or x (conv front end)
  union { const void* k; const uint16_t* conv_w; };
  union { const void* v; const uint16_t* conv_in; };
  uint16_t* conv_out;
  union { const uint16_t* a; const float* alpha; };  // by gate_raw
  union { const uint16_t* b; const float* beta; };
  const float* A_log;
  const float* dt_bias;
  const float* state_in;
  float* state_out;
  void* o;
  // read by the kernel for any T only
  int n_layers, T, nblocks;
  float* states;
};
static_assert(offsetof(RecurrentParams, n_layers) == 128, "the T = 1 fields fill two 64-byte lines");

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
