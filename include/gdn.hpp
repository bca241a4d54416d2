// gdn.hpp -- header-only C++ host layer over the C ABI of libgdn.so (gdn.h).
//
// Mirrors the reference's per-layer C++ interface so a DeltaNet layer can call it where
// it called the Metal kernel (paths relative to the reference tree):
//   gdn::run            delta::run(q, k, v, alpha, beta, S, collect)   cpp/src/delta.hpp:66-68
//   gdn::Layer::step    the recurrent core of GatedDeltaNet::operator(),
//                       front end + gates + delta::run + cache advance  cpp/src/model.cpp:585-638
//   gdn::DeltaCache     DeltaCache with record / commit(n)             cpp/src/model.hpp:211-227,
//                                                                       cpp/src/model.cpp:439-457
//   gdn::linear(s)      Linear::operator(), 4-bit weights              cpp/src/model.cpp:356-372
//   gdn::norm_out_proj  out_proj(GatedRMSNorm(o, z))                   cpp/src/model.cpp:626-641
// Errors are C++ exceptions on this side of the ABI (the reference's fail() /
// std::runtime_error convention); the ABI itself never throws.
//
// Device memory: buffers owned here are allocated once, when a DeltaCache is created,
// never on a step. Every call is ordered on the given stream and does not synchronise.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <utility>

#include "gdn.h"

namespace gdn {

struct Error : std::runtime_error {
  int code;
  Error(int c, const std::string& msg) : std::runtime_error(msg), code(c) {}
};

inline void check(int rc) {
  if (rc != GDN_OK) throw Error(rc, gdn_last_error());
}

inline void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess) throw Error(GDN_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

inline bool available() { return gdn_available() != 0; }

// Blocks of B sequences that are not recorded and carry at least chunked_min_t(B) tokens run
// the chunked form (gdn_prefill_chunked), shorter ones the recurrent kernel: the two meet near
// T = 36, 32, 30 and 32 for B = 1, 2, 4 and 8 on MI355X (one layer, conv front end, the
// accurate chunked precision). The reference chooses by length the same way
// (python/qwen35.py:338, 606-626).
constexpr int kChunkedMinT = 28;
constexpr int chunked_min_t(int B) {
  const int t = B == 1 ? 36 : B == 2 ? 32 : B == 3 ? 31 : B == 4 ? 30 : 32;
  return t > kChunkedMinT ? t : kChunkedMinT;
}

// delta::run (delta.hpp:66-68) on device buffers: q, k (B,L,H,128), v (B,L,H,128), alpha,
// beta (B,L,H), all fp32, head-expanded as the reference passes them; S (B,H,128,128) or
// nullptr for zeros. Writes o (B,L,H,128) fp32, s_out and, when states != nullptr, the
// per-step states (B,H,L,128,128) -- the reference's S_all (delta.cpp:155-171).
inline void run(int B, int L, int H, const float* q, const float* k, const float* v,
                const float* alpha, const float* beta, const float* S, float* o, float* s_out,
                float* states = nullptr, hipStream_t stream = nullptr) {
  gdn_layer_args a{};
  a.n_layers = 1;
  a.batch = B;
  a.seq_len = L;
  a.num_k_heads = H;
  a.num_v_heads = H;
  a.frontend = GDN_FRONTEND_QKV;
  a.q = q;
  a.k = k;
  a.v = v;
  a.qkv_dtype = GDN_DTYPE_F32;
  a.gate_mode = GDN_GATES_PRECOMPUTED;
  a.alpha = alpha;
  a.beta = beta;
  a.state_in = S;
  a.state_out = s_out;
  a.states = states;
  a.states_layout = GDN_STATES_BHT;
  a.o = o;
  a.o_dtype = GDN_DTYPE_F32;
  a.stream = stream;
  check(gdn_run(&a));
}

// One Gated-DeltaNet layer's fixed parameters (device pointers, loaded elsewhere):
// conv1d.weight transposed to (4, C) bf16, A_log and dt_bias (Hv) fp32.
struct LayerParams {
  const void* conv_weight = nullptr;
  const float* A_log = nullptr;
  const float* dt_bias = nullptr;
  int num_k_heads = 16;
  int num_v_heads = 48;
  int conv_dim() const { return 2 * num_k_heads * GDN_HEAD_DIM + num_v_heads * GDN_HEAD_DIM; }
};

// DeltaCache (model.hpp:211-227): the layer's fp32 state and the 3 pre-conv rows, with
// record mode for speculative blocks. The conv rows live in two buffers that swap roles
// every step (the kernel never updates them in place).
class DeltaCache {
 public:
  // Recorded blocks go to two buffers of max_record_steps states each, (T, B, Hv) order,
  // used in turn: commit(n) adopts step n-1 of the block by pointer (no copy), and the
  // next block is recorded into the other buffer, which no longer holds the live state.
  // Blocks of chunked_min_t(batch) .. max_prefill_tokens tokens (the reference prefills in windows of
  // 1024, cpp/src/session.hpp:136) run the chunked form in a workspace allocated here, with
  // `prefill_precision` (gdn_prefill_precision: GDN_PREFILL_ACCURATE, the default, leaves the
  // state the next decode step starts from within about 1e-5 of the fp32 recurrence,
  // GDN_PREFILL_FAST about 2e-3 to 4e-3 in about 0.85 of the time); max_prefill_tokens = 0
  // keeps every block on the exact recurrent kernel.
  DeltaCache(const LayerParams& p, int batch, int max_record_steps, int max_prefill_tokens = 0,
             int prefill_precision = GDN_PREFILL_ACCURATE)
      : p_(p), B_(batch), max_T_(max_record_steps),
        max_prefill_T_(max_prefill_tokens >= chunked_min_t(batch) ? max_prefill_tokens : 0),
        precision_(prefill_precision) {
    const size_t D = GDN_HEAD_DIM;
    state_bytes_ = (size_t)B_ * p_.num_v_heads * D * D * sizeof(float);
    conv_bytes_ = (size_t)B_ * (GDN_CONV_TAPS - 1) * p_.conv_dim() * 2;
    check_hip(hipMalloc(&own_state_, state_bytes_), "hipMalloc state");
    check_hip(hipMalloc(&conv_, conv_bytes_), "hipMalloc conv");
    check_hip(hipMalloc(&conv_spare_, conv_bytes_), "hipMalloc conv");
    for (float*& r : rec_)
      if (max_T_ > 0) check_hip(hipMalloc(&r, state_bytes_ * max_T_), "hipMalloc states");
    if (max_prefill_T_ > 0) {
      gdn_layer_args w{};
      w.batch = B_;
      w.seq_len = max_prefill_T_;
      w.num_k_heads = p_.num_k_heads;
      w.num_v_heads = p_.num_v_heads;
      w.frontend = GDN_FRONTEND_CONV;
      w.prefill_precision = precision_;
      check(gdn_prefill_workspace_size(&w, &ws_bytes_));
      check_hip(hipMalloc(&ws_, ws_bytes_), "hipMalloc prefill workspace");
    }
    check_hip(hipMemset(own_state_, 0, state_bytes_), "hipMemset");
    check_hip(hipMemset(conv_, 0, conv_bytes_), "hipMemset");
    state_ = own_state_;
  }
  DeltaCache(const DeltaCache&) = delete;
  DeltaCache& operator=(const DeltaCache&) = delete;
  ~DeltaCache() {
    (void)hipFree(own_state_);
    (void)hipFree(conv_);
    (void)hipFree(conv_spare_);
    for (float* r : rec_)
      if (r) (void)hipFree(r);
    if (ws_) (void)hipFree(ws_);
  }

  int offset = 0;
  bool record = false;

  // The live state (B, Hv, 128, 128) fp32. After a commit(n > 0) it is a block of a
  // recording buffer, so re-read the pointer after every commit.
  float* state() const { return state_; }
  void* conv() const { return conv_; }
  size_t state_bytes() const { return state_bytes_; }
  size_t conv_bytes() const { return conv_bytes_; }

  // GatedDeltaNet::operator() from the in_proj outputs to o (model.cpp:585-638):
  // x (B,T,C) bf16 = in_proj_qkv(x), a, b (B,T,Hv) bf16 = in_proj_a/b(x); o (B,T,Hv,128)
  // bf16. In record mode the state is not advanced and every per-step state is kept for
  // commit(); x must then stay valid until commit(). A block that is not recorded and has
  // chunked_min_t(B) .. max_prefill_tokens tokens (x and o 16-byte aligned) runs the chunked form.
  void step(const void* x, const void* a, const void* b, int T, void* o, hipStream_t stream) {
    gdn_layer_args g{};
    g.n_layers = 1;
    g.batch = B_;
    g.seq_len = T;
    g.num_k_heads = p_.num_k_heads;
    g.num_v_heads = p_.num_v_heads;
    g.frontend = GDN_FRONTEND_CONV;
    g.x = x;
    g.conv_weight = p_.conv_weight;
    g.conv_state_in = conv_;
    g.gate_mode = GDN_GATES_RAW;
    g.a = a;
    g.b = b;
    g.A_log = p_.A_log;
    g.dt_bias = p_.dt_bias;
    g.state_in = state_;
    g.states_layout = GDN_STATES_TBH;
    g.o = o;
    g.o_dtype = GDN_DTYPE_BF16;
    g.stream = stream;
    if (record) {
      if (T > max_T_) throw Error(GDN_EINVAL, "DeltaCache: record block longer than max_record_steps");
      pending_states_ = holds_state(rec_[0]) ? rec_[1] : rec_[0];
      g.states = pending_states_;
      check(gdn_run(&g));
      base_offset_ = offset;
      pending_x_ = x;
      pending_T_ = T;
    } else {
      g.conv_state_out = conv_spare_;
      g.state_out = state_;
      const bool aligned = (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(o)) % 16 == 0;
      if (T >= chunked_min_t(B_) && T <= max_prefill_T_ && aligned) {
        g.workspace = ws_;
        g.workspace_bytes = ws_bytes_;
        g.prefill_precision = precision_;
        check(gdn_prefill_chunked(&g));
      } else {
        check(gdn_run(&g));
      }
      std::swap(conv_, conv_spare_);
      offset += T;
    }
  }

  // Accept the first n tokens of the recorded block (model.cpp:439-457).
  void commit(int n, hipStream_t stream) {
    if (pending_T_ < 0) return;
    if (n < 0 || n > pending_T_) throw Error(GDN_EINVAL, "DeltaCache::commit out of range");
    gdn_commit_args c{};
    c.n_layers = 1;
    c.batch = B_;
    c.seq_len = pending_T_;
    c.num_v_heads = p_.num_v_heads;
    c.conv_dim = p_.conv_dim();
    c.n = n;
    c.states = pending_states_;
    c.states_layout = GDN_STATES_TBH;
    c.state_prev = state_;
    // pointer swap: step n-1 of the block becomes the state where it lies
    float* adopted = n == 0 ? state_ : pending_states_ + (size_t)(n - 1) * (state_bytes_ / sizeof(float));
    c.state_dst = adopted;
    c.conv_state_in = conv_;
    c.x = pending_x_;
    c.conv_state_dst = conv_;
    c.stream = stream;
    check(gdn_commit(&c));
    state_ = adopted;
    offset = base_offset_ + n;
    pending_T_ = -1;
    pending_x_ = nullptr;
    record = false;
  }

 private:
  LayerParams p_;
  int B_;
  int max_T_;
  int max_prefill_T_;
  int precision_;
  size_t state_bytes_ = 0, conv_bytes_ = 0, ws_bytes_ = 0;
  void* ws_ = nullptr;
  bool holds_state(const float* rec) const {
    const uintptr_t s = reinterpret_cast<uintptr_t>(state_), r = reinterpret_cast<uintptr_t>(rec);
    return rec && s >= r && s < r + state_bytes_ * (size_t)max_T_;
  }

  float* own_state_ = nullptr;
  float* state_ = nullptr;  // own_state_ or a block of rec_[0] / rec_[1]
  void* conv_ = nullptr;
  void* conv_spare_ = nullptr;
  float* rec_[2] = {nullptr, nullptr};
  float* pending_states_ = nullptr;
  int base_offset_ = 0;
  const void* pending_x_ = nullptr;
  int pending_T_ = -1;
};

// Linear::operator() for the reference's 4-bit weights (cpp/src/model.cpp:356-372), on
// device pointers in the checkpoint's layout: w (N, K/8) uint32, scales and biases
// (N, K/64) bf16.
struct QuantLinear {
  const void* w = nullptr;
  const void* scales = nullptr;
  const void* biases = nullptr;
  int n = 0;  // out features
};

// Workspace bytes the projections below need for M rows of K (0 up to
// GDN_QLINEAR_GEMV_ROWS rows: the GEMV kernel; more rows run on MFMA).
inline size_t qlinear_workspace_size(int M, int K) {
  gdn_qlinear_args a{};
  a.n_layers = 1;
  a.m = M;
  a.k = K;
  size_t n = 0;
  check(gdn_qlinear_workspace_size(&a, &n));
  return n;
}

// y[i] (M, W[i].n) bf16 = x (M, K) bf16 times W[i]^T, for count <= GDN_QLINEAR_MAX_SEGS
// matrices sharing x in one launch -- the layer's in_proj_qkv, in_proj_z, in_proj_a,
// in_proj_b (model.cpp:587, 608-609, 626). More than GDN_QLINEAR_GEMV_ROWS rows need a
// workspace of qlinear_workspace_size(M, K) bytes.
inline void linears(int M, int K, const void* x, const QuantLinear* W, void* const* y, int count,
                    hipStream_t stream = nullptr, void* workspace = nullptr, size_t workspace_bytes = 0) {
  gdn_qlinear_args a{};
  a.n_layers = 1;
  a.m = M;
  a.k = K;
  a.x = x;
  a.n_segs = count;
  for (int i = 0; i < count && i < GDN_QLINEAR_MAX_SEGS; ++i)
    a.segs[i] = gdn_qlinear_seg{W[i].w, W[i].scales, W[i].biases, y[i], W[i].n};
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.stream = stream;
  check(gdn_qlinear(&a));
}

inline void linear(const QuantLinear& W, int M, int K, const void* x, void* y, hipStream_t stream = nullptr,
                   void* workspace = nullptr, size_t workspace_bytes = 0) {
  linears(M, K, x, &W, &y, 1, stream, workspace, workspace_bytes);
}

// out_proj(GatedRMSNorm(o, z)) (model.cpp:626-641): o (M, K) fp32 recurrence output, z (M,
// K) bf16, gamma (128) fp32 -> y (M, W.n) bf16.
inline void norm_out_proj(const QuantLinear& W, int M, int K, const float* o, const void* z, const float* gamma,
                          float eps, void* y, hipStream_t stream = nullptr, void* workspace = nullptr,
                          size_t workspace_bytes = 0) {
  gdn_qlinear_args a{};
  a.n_layers = 1;
  a.m = M;
  a.k = K;
  a.norm_x = o;
  a.norm_z = z;
  a.norm_gamma = gamma;
  a.norm_eps = eps;
  a.n_segs = 1;
  a.segs[0] = gdn_qlinear_seg{W.w, W.scales, W.biases, y, W.n};
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.stream = stream;
  check(gdn_qlinear(&a));
}

}  // namespace gdn
