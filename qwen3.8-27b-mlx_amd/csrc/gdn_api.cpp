// C ABI entry points of libgdn.so: argument validation, device check, dispatch.
//
// Validation runs before any HIP call, so every argument error is reported the same
// way with or without a GPU. No entry point allocates device memory or synchronises.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/gdn.h"
#include "gdn_internal.h"

namespace gdn {
int recurrent_tile_rows(long long heads);
size_t prefill_workspace_bytes(int B, int T, int Hk, int Hv);
hipError_t launch_chunked_prefill(const gdn_layer_args& a, void* workspace, hipStream_t stream,
                                  hipEvent_t* events);
}  // namespace gdn

namespace {

thread_local std::string g_error;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int ok() {
  g_error.clear();
  return GDN_OK;
}

struct Range {
  uintptr_t lo = 0, hi = 0;  // [lo, hi)
  bool empty() const { return lo == hi; }
};

Range range_of(const void* p, int64_t bytes) {
  Range r;
  if (p && bytes > 0) {
    r.lo = reinterpret_cast<uintptr_t>(p);
    r.hi = r.lo + static_cast<uintptr_t>(bytes);
  }
  return r;
}

bool overlap(Range a, Range b) { return !a.empty() && !b.empty() && a.lo < b.hi && b.lo < a.hi; }

bool aligned(const void* p, uintptr_t n) { return (reinterpret_cast<uintptr_t>(p) % n) == 0; }

constexpr int kMaxDevices = 64;
std::once_flag g_dev_once[kMaxDevices];
int g_dev_ok[kMaxDevices];  // 1 = gfx950, 0 = other, -1 = query failed
std::string g_dev_name[kMaxDevices];

// Checks the current device once per device (lazily, thread-safe).
int check_device() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(GDN_EDEVICE, "hipGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(GDN_EDEVICE, "device index %d out of range", dev);
  std::call_once(g_dev_once[dev], [dev] {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
      g_dev_ok[dev] = -1;
      return;
    }
    g_dev_name[dev] = prop.gcnArchName;
    g_dev_ok[dev] = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
  });
  if (g_dev_ok[dev] < 0) return fail(GDN_EDEVICE, "hipGetDeviceProperties failed on device %d", dev);
  if (g_dev_ok[dev] == 0) {
    return fail(GDN_EUNSUPPORTED, "device %d is %s; libgdn is built for gfx950 only", dev,
                g_dev_name[dev].c_str());
  }
  return GDN_OK;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(GDN_EDEVICE, "%s: %s", what, hipGetErrorString(e));
}

// Shared validation of gdn_run / gdn_prefill_chunked. Fills the per-layer element
// counts used for the overlap checks.
int validate_layer(const gdn_layer_args* a, const char* fn, bool allow_states) {
  if (!a) return fail(GDN_EINVAL, "%s: args is NULL", fn);
  if (a->n_layers < 1) return fail(GDN_EINVAL, "%s: n_layers must be >= 1 (got %d)", fn, a->n_layers);
  if (a->batch < 0) return fail(GDN_EINVAL, "%s: batch must be >= 0 (got %d)", fn, a->batch);
  if (a->seq_len < 0) return fail(GDN_EINVAL, "%s: seq_len must be >= 0 (got %d)", fn, a->seq_len);
  if (a->num_k_heads < 1 || a->num_v_heads < 1)
    return fail(GDN_EINVAL, "%s: head counts must be >= 1 (Hk=%d, Hv=%d)", fn, a->num_k_heads,
                a->num_v_heads);
  if (a->num_v_heads % a->num_k_heads != 0)
    return fail(GDN_EINVAL, "%s: num_v_heads (%d) must be a multiple of num_k_heads (%d)", fn,
                a->num_v_heads, a->num_k_heads);
  if (a->frontend != GDN_FRONTEND_QKV && a->frontend != GDN_FRONTEND_CONV)
    return fail(GDN_EINVAL, "%s: unknown frontend %d", fn, a->frontend);
  if (a->gate_mode != GDN_GATES_RAW && a->gate_mode != GDN_GATES_PRECOMPUTED)
    return fail(GDN_EINVAL, "%s: unknown gate_mode %d", fn, a->gate_mode);
  if (a->o_dtype != GDN_DTYPE_BF16 && a->o_dtype != GDN_DTYPE_F32)
    return fail(GDN_EINVAL, "%s: unknown o_dtype %d", fn, a->o_dtype);
  if (a->frontend == GDN_FRONTEND_QKV && a->qkv_dtype != GDN_DTYPE_BF16 &&
      a->qkv_dtype != GDN_DTYPE_F32)
    return fail(GDN_EINVAL, "%s: unknown qkv_dtype %d", fn, a->qkv_dtype);
  if (a->states_layout != GDN_STATES_BHT && a->states_layout != GDN_STATES_TBH)
    return fail(GDN_EINVAL, "%s: unknown states_layout %d", fn, a->states_layout);
  if (a->prefill_precision != GDN_PREFILL_FAST && a->prefill_precision != GDN_PREFILL_ACCURATE)
    return fail(GDN_EINVAL, "%s: unknown prefill_precision %d", fn, a->prefill_precision);
  if (!allow_states && a->states)
    return fail(GDN_EINVAL, "%s: per-step states are not produced by this entry point", fn);

  const int64_t L = a->n_layers, B = a->batch, T = a->seq_len, Hk = a->num_k_heads,
                Hv = a->num_v_heads, D = GDN_HEAD_DIM;
  // every element count must fit comfortably in int64 and the grid in int32
  if (L * B * Hv > (int64_t)1 << 28)
    return fail(GDN_EINVAL, "%s: n_layers*batch*num_v_heads too large", fn);
  if (L * B * T > (int64_t)1 << 31) return fail(GDN_EINVAL, "%s: n_layers*batch*seq_len too large", fn);
  if (B == 0) return GDN_OK;

  const int64_t C = 2 * Hk * D + Hv * D;
  const int64_t state_b = L * B * Hv * D * D * 4;
  const int64_t ob = L * B * T * Hv * D * (a->o_dtype == GDN_DTYPE_BF16 ? 2 : 4);

  if (a->frontend == GDN_FRONTEND_QKV) {
    if (T > 0 && (!a->q || !a->k || !a->v))
      return fail(GDN_EINVAL, "%s: q, k and v are required by the qkv front end", fn);
    const uintptr_t al = a->qkv_dtype == GDN_DTYPE_BF16 ? 2 : 4;
    if (!aligned(a->q, al) || !aligned(a->k, al) || !aligned(a->v, al))
      return fail(GDN_EINVAL, "%s: q, k, v must be aligned to their element size", fn);
  } else {
    if (T > 0 && !a->x) return fail(GDN_EINVAL, "%s: x is required by the conv front end", fn);
    if (!a->conv_weight) return fail(GDN_EINVAL, "%s: conv_weight is required by the conv front end", fn);
    if (!aligned(a->x, 2) || !aligned(a->conv_weight, 2) || !aligned(a->conv_state_in, 2) ||
        !aligned(a->conv_state_out, 2))
      return fail(GDN_EINVAL, "%s: conv tensors must be 2-byte aligned", fn);
    const Range cout = range_of(a->conv_state_out, L * B * 3 * C * 2);
    if (overlap(cout, range_of(a->conv_state_in, L * B * 3 * C * 2)))
      return fail(GDN_EINVAL, "%s: conv_state_out must not overlap conv_state_in", fn);
    if (overlap(cout, range_of(a->x, L * B * T * C * 2)) ||
        overlap(cout, range_of(a->conv_weight, L * 4 * C * 2)))
      return fail(GDN_EINVAL, "%s: conv_state_out must not overlap x or conv_weight", fn);
  }
  if (T > 0) {
    if (a->gate_mode == GDN_GATES_RAW) {
      if (!a->a || !a->b || !a->A_log || !a->dt_bias)
        return fail(GDN_EINVAL, "%s: a, b, A_log and dt_bias are required for raw gates", fn);
      if (!aligned(a->a, 2) || !aligned(a->b, 2) || !aligned(a->A_log, 4) || !aligned(a->dt_bias, 4))
        return fail(GDN_EINVAL, "%s: gate tensors must be aligned to their element size", fn);
    } else {
      if (!a->alpha || !a->beta)
        return fail(GDN_EINVAL, "%s: alpha and beta are required for precomputed gates", fn);
      if (!aligned(a->alpha, 4) || !aligned(a->beta, 4))
        return fail(GDN_EINVAL, "%s: alpha and beta must be 4-byte aligned", fn);
    }
    if (!a->o) return fail(GDN_EINVAL, "%s: o is required", fn);
    if (!aligned(a->o, a->o_dtype == GDN_DTYPE_BF16 ? 2 : 4))
      return fail(GDN_EINVAL, "%s: o must be aligned to its element size", fn);
  }
  if (!aligned(a->state_in, 16) || !aligned(a->state_out, 16) || !aligned(a->states, 16))
    return fail(GDN_EINVAL, "%s: state buffers must be 16-byte aligned", fn);
  const Range sin = range_of(a->state_in, state_b);
  const Range sout = range_of(a->state_out, state_b);
  const Range sts = range_of(a->states, state_b * T);
  if (overlap(sin, sout) && a->state_in != a->state_out)
    return fail(GDN_EINVAL, "%s: state_out must equal state_in or not overlap it", fn);
  if (overlap(sts, sin)) return fail(GDN_EINVAL, "%s: states must not overlap state_in", fn);
  if (overlap(sts, sout)) return fail(GDN_EINVAL, "%s: states must not overlap state_out", fn);
  const Range orng = range_of(a->o, ob);
  if (overlap(orng, sin) || overlap(orng, sout) || overlap(orng, sts))
    return fail(GDN_EINVAL, "%s: o must not overlap the state buffers", fn);
  return GDN_OK;
}

// An empty block (T = 0): state_out <- state_in, conv_state_out <- conv_state_in.
int run_empty(const gdn_layer_args* a, hipStream_t stream) {
  const int64_t L = a->n_layers, B = a->batch, Hk = a->num_k_heads, Hv = a->num_v_heads,
                D = GDN_HEAD_DIM;
  if (a->state_out && a->state_out != a->state_in) {
    hipError_t e = gdn::launch_copy_f32(a->state_out, a->state_in, L * B * Hv * D * D, stream);
    if (e != hipSuccess) return hip_fail(e, "copy kernel");
  }
  if (a->frontend == GDN_FRONTEND_CONV && a->conv_state_out) {
    const int64_t C = 2 * Hk * D + Hv * D;
    hipError_t e = gdn::launch_copy_u16(static_cast<uint16_t*>(a->conv_state_out),
                                        static_cast<const uint16_t*>(a->conv_state_in),
                                        L * B * 3 * C, stream);
    if (e != hipSuccess) return hip_fail(e, "copy kernel");
  }
  return ok();
}

// Shared validation of gdn_qlinear / gdn_qlinear_noalloc. With `noalloc` the workspace
// fields must be empty and the MFMA path's operand must fit the library's scratch (which no
// caller buffer can overlap: its address is not exposed).
int validate_qlinear(const gdn_qlinear_args* a, const char* fn, bool noalloc) {
  if (!a) return fail(GDN_EINVAL, "%s: args is NULL", fn);
  if (a->n_layers < 1 || a->m < 1 || a->m > GDN_QLINEAR_MAX_ROWS)
    return fail(GDN_EINVAL, "%s: bad shape (n_layers=%d m=%d; m must be 1..%d)", fn, a->n_layers, a->m,
                GDN_QLINEAR_MAX_ROWS);
  if (!gdn::qlinear_k_supported(a->k))
    return fail(GDN_EINVAL, "%s: k=%d unsupported (1024, 2048, 4096, 5120, 6144, 8192)", fn, a->k);
  if (a->n_segs < 1 || a->n_segs > GDN_QLINEAR_MAX_SEGS)
    return fail(GDN_EINVAL, "%s: n_segs must be 1..%d", fn, GDN_QLINEAR_MAX_SEGS);
  const int64_t L = a->n_layers, M = a->m, K = a->k;
  const size_t ws_need = gdn::qlinear_workspace_bytes(a->n_layers, a->m, a->k);
  if (noalloc) {
    if (a->workspace || a->workspace_bytes)
      return fail(GDN_EINVAL, "%s: takes no workspace (workspace must be NULL, workspace_bytes 0)", fn);
    if (ws_need > GDN_QLINEAR_NOALLOC_SCRATCH_BYTES)
      return fail(GDN_EINVAL, "%s: n_layers=%d m=%d k=%d needs %zu bytes of scratch, more than the %zu the library holds",
                  fn, a->n_layers, a->m, a->k, ws_need, (size_t)GDN_QLINEAR_NOALLOC_SCRATCH_BYTES);
  } else if (ws_need > 0) {  // MFMA path: the operand in fragment order goes to the workspace
    if (!a->workspace || a->workspace_bytes < ws_need)
      return fail(GDN_EINVAL, "%s: m=%d k=%d needs a workspace of %zu bytes (got %zu)", fn, a->m, a->k, ws_need,
                  a->workspace ? a->workspace_bytes : (size_t)0);
    if (!aligned(a->workspace, 256)) return fail(GDN_EINVAL, "%s: workspace must be 256-byte aligned", fn);
  }
  const bool norm = a->norm_x != nullptr;
  if (norm == (a->x != nullptr))
    return fail(GDN_EINVAL, "%s: exactly one of x and norm_x is required", fn);
  Range in[3];
  if (norm) {
    if (!a->norm_z || !a->norm_gamma) return fail(GDN_EINVAL, "%s: the norm needs norm_z and norm_gamma", fn);
    if (!(a->norm_eps >= 0.0f)) return fail(GDN_EINVAL, "%s: norm_eps must be >= 0", fn);
    if (!aligned(a->norm_x, 16) || !aligned(a->norm_z, 16) || !aligned(a->norm_gamma, 16))
      return fail(GDN_EINVAL, "%s: norm_x, norm_z and norm_gamma must be 16-byte aligned", fn);
    in[0] = range_of(a->norm_x, L * M * K * 4);
    in[1] = range_of(a->norm_z, L * M * K * 2);
    in[2] = range_of(a->norm_gamma, L * 128 * 4);
  } else {
    if (!aligned(a->x, 16)) return fail(GDN_EINVAL, "%s: x must be 16-byte aligned", fn);
    in[0] = range_of(a->x, L * M * K * 2);
  }
  int64_t rows = 0;
  for (int i = 0; i < a->n_segs; ++i) {
    const gdn_qlinear_seg& g = a->segs[i];
    if (!g.w || !g.scales || !g.biases || !g.y || g.n < 1)
      return fail(GDN_EINVAL, "%s: segment %d needs w, scales, biases, y and n >= 1", fn, i);
    if (!aligned(g.w, 16) || !aligned(g.scales, 8) || !aligned(g.biases, 8) || !aligned(g.y, 2))
      return fail(GDN_EINVAL, "%s: segment %d: w must be 16-byte, scales and biases 8-byte and y 2-byte aligned", fn, i);
    rows += g.n;
  }
  if (rows * L > (int64_t)1 << 31) return fail(GDN_EINVAL, "%s: too many rows", fn);
  const Range ws = range_of(ws_need > 0 && !noalloc ? a->workspace : nullptr, (int64_t)ws_need);
  for (const Range& r : in)
    if (overlap(ws, r)) return fail(GDN_EINVAL, "%s: the workspace must not overlap the operand", fn);
  for (int i = 0; i < a->n_segs; ++i) {
    const gdn_qlinear_seg& g = a->segs[i];
    const Range y = range_of(g.y, L * M * g.n * 2);
    if (overlap(y, ws)) return fail(GDN_EINVAL, "%s: segment %d: y must not overlap the workspace", fn, i);
    if (overlap(ws, range_of(g.w, L * g.n * K / 2)) || overlap(ws, range_of(g.scales, L * g.n * K / 32)) ||
        overlap(ws, range_of(g.biases, L * g.n * K / 32)))
      return fail(GDN_EINVAL, "%s: the workspace must not overlap segment %d's weights", fn, i);
    for (const Range& r : in)
      if (overlap(y, r)) return fail(GDN_EINVAL, "%s: segment %d: y must not overlap the operand", fn, i);
    for (int j = 0; j < a->n_segs; ++j) {
      const gdn_qlinear_seg& h = a->segs[j];
      if (overlap(y, range_of(h.w, L * h.n * K / 2)) || overlap(y, range_of(h.scales, L * h.n * K / 32)) ||
          overlap(y, range_of(h.biases, L * h.n * K / 32)))
        return fail(GDN_EINVAL, "%s: segment %d: y must not overlap a weight tensor", fn, i);
      if (j != i && overlap(y, range_of(h.y, L * M * h.n * 2)))
        return fail(GDN_EINVAL, "%s: outputs of segments %d and %d overlap", fn, i, j);
    }
  }
  return GDN_OK;
}

}  // namespace

extern "C" {

int gdn_abi_version(void) { return GDN_ABI_VERSION; }

const char* gdn_last_error(void) { return g_error.c_str(); }

int gdn_available(void) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess) return 0;
  return std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
}

int gdn_run(const gdn_layer_args* a) {
  int rc = validate_layer(a, "gdn_run", true);
  if (rc != GDN_OK) return rc;
  if (a->batch == 0) return ok();
  rc = check_device();
  if (rc != GDN_OK) return rc;
  hipStream_t stream = static_cast<hipStream_t>(a->stream);
  if (a->seq_len == 0) return run_empty(a, stream);

  gdn::RecurrentParams p{};
  p.n_layers = a->n_layers;
  p.B = a->batch;
  p.T = a->seq_len;
  p.Hk = a->num_k_heads;
  p.Hv = a->num_v_heads;
  p.rep = p.Hv / p.Hk;
  p.C = 2 * p.Hk * GDN_HEAD_DIM + p.Hv * GDN_HEAD_DIM;
  p.qkv_bf16 = a->qkv_dtype == GDN_DTYPE_BF16;
  p.gate_raw = a->gate_mode == GDN_GATES_RAW;
  p.o_bf16 = a->o_dtype == GDN_DTYPE_BF16;
  p.states_tbh = a->states_layout == GDN_STATES_TBH;
  const int64_t tiles =
      GDN_HEAD_DIM / gdn::recurrent_tile_rows((long long)a->n_layers * a->batch * a->num_v_heads);
  const int64_t nblocks = (int64_t)a->n_layers * a->batch * a->num_v_heads * tiles;
  p.nblocks = static_cast<int>(nblocks);
  // XCD order: the contiguous split (each XCD one eighth of the grid) for large grids,
  // measured faster from B = 8 at 48 layers (36,864 workgroups: 407 vs 418 us; B = 16: 821
  // vs 865 us) and slower for smaller ones (B = 1 over 8 state sets: 56.2 vs 53.2 us), which
  // interleave k-head groups over the XCDs instead (B = 1: 53.6 -> 52.9 us).
  const bool split = (nblocks % 8) == 0 && nblocks > 16384;
  const int64_t grp8 = 8 * (int64_t)p.rep * tiles;  // workgroups of 8 k-heads
  p.order = split ? 1 : (nblocks % grp8 == 0 ? 2 : 0);
  // The block map's quotients n / d (n < nblocks) as multiply-highs by ceil(2^32 / d): exact
  // when n d <= 2^32 (the error n (d ceil(2^32 / d) - 2^32) / d 2^32 stays below 1 / d).
  auto recip = [](int64_t d) -> uint32_t { return d == 1 ? 0u : (uint32_t)(((1ull << 32) + d - 1) / d); };
  const int64_t dmax = std::max(std::max(grp8, (int64_t)p.Hv), std::max((int64_t)p.B, (int64_t)p.rep));
  p.fastdiv = nblocks * dmax <= (1ll << 32);
  p.rc_grp8 = recip(grp8);
  p.rc_hv = recip(p.Hv);
  p.rc_b = recip(p.B);
  p.rc_rep = recip(p.rep);
  if (a->frontend == GDN_FRONTEND_CONV) {
    p.x = static_cast<const uint16_t*>(a->x);
    p.conv_w = static_cast<const uint16_t*>(a->conv_weight);
    p.conv_in = static_cast<const uint16_t*>(a->conv_state_in);
    p.conv_out = static_cast<uint16_t*>(a->conv_state_out);
  } else {
    p.q = a->q;
    p.k = a->k;
    p.v = a->v;
  }
  if (p.gate_raw) {
    p.a = static_cast<const uint16_t*>(a->a);
    p.b = static_cast<const uint16_t*>(a->b);
    p.A_log = a->A_log;
    p.dt_bias = a->dt_bias;
  } else {
    p.alpha = a->alpha;
    p.beta = a->beta;
  }
  p.state_in = a->state_in;
  p.state_out = a->state_out;
  p.states = a->states;
  p.o = a->o;
  hipError_t e = gdn::launch_recurrent(p, a->frontend, a->states != nullptr, stream);
  if (e != hipSuccess) return hip_fail(e, "gdn_run launch");
  return ok();
}

int gdn_prefill_workspace_size(const gdn_layer_args* a, size_t* bytes) {
  if (!a || !bytes) return fail(GDN_EINVAL, "gdn_prefill_workspace_size: NULL argument");
  if (a->batch < 0 || a->seq_len < 0 || a->num_k_heads < 1 || a->num_v_heads < 1)
    return fail(GDN_EINVAL, "gdn_prefill_workspace_size: bad shape");
  if (a->prefill_precision != GDN_PREFILL_FAST && a->prefill_precision != GDN_PREFILL_ACCURATE)
    return fail(GDN_EINVAL, "gdn_prefill_workspace_size: unknown prefill_precision %d", a->prefill_precision);
  *bytes = gdn::prefill_workspace_bytes(a->batch, a->seq_len, a->num_k_heads, a->num_v_heads);
  return ok();
}

namespace {

// The argument checks of gdn_prefill_chunked (no HIP call).
int prefill_validate(const gdn_layer_args* a) {
  int rc = validate_layer(a, "gdn_prefill_chunked", false);
  if (rc != GDN_OK) return rc;
  if (a->batch == 0) return ok();
  if (a->frontend == GDN_FRONTEND_QKV && a->qkv_dtype != GDN_DTYPE_BF16)
    return fail(GDN_EINVAL, "gdn_prefill_chunked: the qkv front end takes bf16 q, k, v");
  if (a->frontend == GDN_FRONTEND_CONV && (!aligned(a->x, 16) || !aligned(a->conv_state_in, 16)))
    return fail(GDN_EINVAL, "gdn_prefill_chunked: x and conv_state_in must be 16-byte aligned");
  if (a->frontend == GDN_FRONTEND_QKV && (!aligned(a->q, 16) || !aligned(a->k, 16) || !aligned(a->v, 16)))
    return fail(GDN_EINVAL, "gdn_prefill_chunked: q, k and v must be 16-byte aligned");
  if (!aligned(a->o, 16)) return fail(GDN_EINVAL, "gdn_prefill_chunked: o must be 16-byte aligned");
  const size_t need = gdn::prefill_workspace_bytes(a->batch, a->seq_len, a->num_k_heads, a->num_v_heads);
  if (a->seq_len > 0) {
    if (!a->workspace || a->workspace_bytes < need)
      return fail(GDN_EINVAL, "gdn_prefill_chunked: workspace of %zu bytes required (got %zu)", need,
                  a->workspace ? a->workspace_bytes : (size_t)0);
    if (!aligned(a->workspace, 256))
      return fail(GDN_EINVAL, "gdn_prefill_chunked: workspace must be 256-byte aligned");
    const int64_t L = a->n_layers;
    if (L != 1) return fail(GDN_EINVAL, "gdn_prefill_chunked: one layer per call (n_layers = 1)");
    // the workspace is written while every other buffer is read or written
    const int64_t B = a->batch, T = a->seq_len, Hk = a->num_k_heads, Hv = a->num_v_heads,
                  D = GDN_HEAD_DIM, C = 2 * Hk * D + Hv * D;
    const bool conv = a->frontend == GDN_FRONTEND_CONV, raw = a->gate_mode == GDN_GATES_RAW;
    const struct {
      const void* p;
      int64_t bytes;
      const char* name;
    } bufs[] = {
        {a->o, B * T * Hv * D * (a->o_dtype == GDN_DTYPE_BF16 ? 2 : 4), "o"},
        {a->state_in, B * Hv * D * D * 4, "state_in"},
        {a->state_out, B * Hv * D * D * 4, "state_out"},
        {conv ? a->x : nullptr, B * T * C * 2, "x"},
        {conv ? a->conv_weight : nullptr, 4 * C * 2, "conv_weight"},
        {conv ? a->conv_state_in : nullptr, B * 3 * C * 2, "conv_state_in"},
        {conv ? a->conv_state_out : nullptr, B * 3 * C * 2, "conv_state_out"},
        {conv ? nullptr : a->q, B * T * Hk * D * 2, "q"},
        {conv ? nullptr : a->k, B * T * Hk * D * 2, "k"},
        {conv ? nullptr : a->v, B * T * Hv * D * 2, "v"},
        {raw ? a->a : nullptr, B * T * Hv * 2, "a"},
        {raw ? a->b : nullptr, B * T * Hv * 2, "b"},
        {raw ? a->A_log : nullptr, Hv * 4, "A_log"},
        {raw ? a->dt_bias : nullptr, Hv * 4, "dt_bias"},
        {raw ? nullptr : a->alpha, B * T * Hv * 4, "alpha"},
        {raw ? nullptr : a->beta, B * T * Hv * 4, "beta"},
    };
    const Range ws = range_of(a->workspace, (int64_t)need);
    for (const auto& buf : bufs)
      if (overlap(ws, range_of(buf.p, buf.bytes)))
        return fail(GDN_EINVAL, "gdn_prefill_chunked: the workspace must not overlap %s", buf.name);
  }
  return ok();
}

// The launches of gdn_prefill_chunked for validated arguments; with `events` (four, when
// the call launches the three kernels), an event is recorded before the first kernel and
// after each.
int prefill_launch(const gdn_layer_args* a, hipEvent_t* events) {
  if (a->batch == 0) return ok();
  int rc = check_device();
  if (rc != GDN_OK) return rc;
  hipStream_t stream = static_cast<hipStream_t>(a->stream);
  if (a->seq_len == 0) return run_empty(a, stream);
  hipError_t e = gdn::launch_chunked_prefill(*a, a->workspace, stream, events);
  if (e != hipSuccess) return hip_fail(e, "gdn_prefill_chunked launch");
  return ok();
}

}  // namespace

int gdn_prefill_chunked(const gdn_layer_args* a) {
  const int rc = prefill_validate(a);
  return rc != GDN_OK ? rc : prefill_launch(a, nullptr);
}

int gdn_prefill_chunked_timed(const gdn_layer_args* a, float* kernel_ms) {
  if (!kernel_ms) return fail(GDN_EINVAL, "gdn_prefill_chunked_timed: kernel_ms is NULL");
  for (int i = 0; i < 3; ++i) kernel_ms[i] = 0.0f;
  int rc = prefill_validate(a);
  if (rc != GDN_OK) return rc;
  if (a->batch == 0 || a->seq_len == 0) return prefill_launch(a, nullptr);
  rc = check_device();
  if (rc != GDN_OK) return rc;
  hipEvent_t ev[4] = {};
  for (int i = 0; i < 4; ++i) {
    const hipError_t e = hipEventCreate(&ev[i]);
    if (e != hipSuccess) {
      for (int j = 0; j < i; ++j) (void)hipEventDestroy(ev[j]);
      return hip_fail(e, "gdn_prefill_chunked_timed: hipEventCreate");
    }
  }
  rc = prefill_launch(a, ev);
  hipError_t e = hipSuccess;
  if (rc == GDN_OK) e = hipEventSynchronize(ev[3]);
  for (int i = 0; rc == GDN_OK && e == hipSuccess && i < 3; ++i) e = hipEventElapsedTime(&kernel_ms[i], ev[i], ev[i + 1]);
  for (int i = 0; i < 4; ++i) (void)hipEventDestroy(ev[i]);
  if (rc == GDN_OK && e != hipSuccess) return hip_fail(e, "gdn_prefill_chunked_timed: events");
  return rc;
}

int gdn_commit(const gdn_commit_args* a) {
  if (!a) return fail(GDN_EINVAL, "gdn_commit: args is NULL");
  if (a->n_layers < 1 || a->batch < 0 || a->seq_len < 0 || a->num_v_heads < 1 || a->conv_dim < 0)
    return fail(GDN_EINVAL, "gdn_commit: bad shape (n_layers=%d batch=%d seq_len=%d Hv=%d C=%d)",
                a->n_layers, a->batch, a->seq_len, a->num_v_heads, a->conv_dim);
  if (a->n < 0 || a->n > a->seq_len)
    return fail(GDN_EINVAL, "gdn_commit: n=%d outside [0, %d] (DeltaCache::commit out of range)",
                a->n, a->seq_len);
  if (a->states_layout != GDN_STATES_BHT && a->states_layout != GDN_STATES_TBH)
    return fail(GDN_EINVAL, "gdn_commit: unknown states_layout %d", a->states_layout);
  if (a->batch == 0) return ok();
  if (!a->state_dst) return fail(GDN_EINVAL, "gdn_commit: state_dst is required");
  if (a->n == 0 && !a->state_prev) return fail(GDN_EINVAL, "gdn_commit: state_prev is required for n = 0");
  if (a->n > 0 && !a->states) return fail(GDN_EINVAL, "gdn_commit: states is required for n > 0");
  if (!aligned(a->states, 16) || !aligned(a->state_prev, 16) || !aligned(a->state_dst, 16))
    return fail(GDN_EINVAL, "gdn_commit: state buffers must be 16-byte aligned");
  const int64_t L = a->n_layers, B = a->batch, T = a->seq_len, Hv = a->num_v_heads,
                D = GDN_HEAD_DIM, C = a->conv_dim;
  const int64_t state_b = L * B * Hv * D * D * 4;
  const Range dst = range_of(a->state_dst, state_b);
  if (a->n > 0 && overlap(dst, range_of(a->states, state_b * T))) {
    // adopting step n-1 in place is the pointer-swap case: allowed only when dst IS that step
    const bool tbh = a->states_layout == GDN_STATES_TBH;
    const float* step = a->states + (tbh ? (int64_t)(a->n - 1) * B * Hv * D * D : 0);
    if (!(tbh && L == 1 && step == a->state_dst))
      return fail(GDN_EINVAL, "gdn_commit: state_dst overlaps states");
  }
  if (a->n == 0 && a->state_prev != a->state_dst && overlap(dst, range_of(a->state_prev, state_b)))
    return fail(GDN_EINVAL, "gdn_commit: state_dst must equal state_prev or not overlap it");
  if (C > 0 && a->conv_state_dst) {
    if (T > 0 && !a->x) return fail(GDN_EINVAL, "gdn_commit: x is required for the conv window");
    if (!aligned(a->x, 2) || !aligned(a->conv_state_in, 2) || !aligned(a->conv_state_dst, 2))
      return fail(GDN_EINVAL, "gdn_commit: conv tensors must be 2-byte aligned");
    const Range cd = range_of(a->conv_state_dst, L * B * 3 * C * 2);
    if (overlap(cd, range_of(a->x, L * B * T * C * 2)))
      return fail(GDN_EINVAL, "gdn_commit: conv_state_dst must not overlap x");
    if (a->conv_state_dst != a->conv_state_in && overlap(cd, range_of(a->conv_state_in, L * B * 3 * C * 2)))
      return fail(GDN_EINVAL, "gdn_commit: conv_state_dst must equal conv_state_in or not overlap it");
  }
  int rc = check_device();
  if (rc != GDN_OK) return rc;
  gdn::CommitParams p{};
  p.n_layers = a->n_layers;
  p.B = a->batch;
  p.T = a->seq_len;
  p.Hv = a->num_v_heads;
  p.C = a->conv_state_dst ? a->conv_dim : 0;
  p.n = a->n;
  p.states_tbh = a->states_layout == GDN_STATES_TBH;
  p.states = a->states;
  p.state_prev = a->state_prev;
  p.state_dst = a->state_dst;
  p.conv_in = static_cast<const uint16_t*>(a->conv_state_in);
  p.x = static_cast<const uint16_t*>(a->x);
  p.conv_dst = static_cast<uint16_t*>(a->conv_state_dst);
  hipError_t e = gdn::launch_commit(p, static_cast<hipStream_t>(a->stream));
  if (e != hipSuccess) return hip_fail(e, "gdn_commit launch");
  return ok();
}

int gdn_qlinear(const gdn_qlinear_args* a) {
  int rc = validate_qlinear(a, "gdn_qlinear", false);
  if (rc != GDN_OK) return rc;
  rc = check_device();
  if (rc != GDN_OK) return rc;
  hipError_t e = gdn::launch_qlinear(*a, static_cast<hipStream_t>(a->stream));
  if (e != hipSuccess) return hip_fail(e, "gdn_qlinear launch");
  return ok();
}

int gdn_qlinear_noalloc(const gdn_qlinear_args* a) {
  int rc = validate_qlinear(a, "gdn_qlinear_noalloc", true);
  if (rc != GDN_OK) return rc;
  rc = check_device();
  if (rc != GDN_OK) return rc;
  gdn_qlinear_args b = *a;
  if (gdn::qlinear_workspace_bytes(a->n_layers, a->m, a->k) > 0) {
    hipError_t e = gdn::qlinear_scratch(&b.workspace);
    if (e != hipSuccess) return hip_fail(e, "gdn_qlinear_noalloc: hipGetSymbolAddress of the scratch");
    b.workspace_bytes = GDN_QLINEAR_NOALLOC_SCRATCH_BYTES;
  }
  hipError_t e = gdn::launch_qlinear(b, static_cast<hipStream_t>(a->stream));
  if (e != hipSuccess) return hip_fail(e, "gdn_qlinear_noalloc launch");
  return ok();
}

int gdn_qlinear_workspace_size(const gdn_qlinear_args* a, size_t* bytes) {
  if (!a || !bytes) return fail(GDN_EINVAL, "gdn_qlinear_workspace_size: NULL argument");
  if (a->n_layers < 1 || a->m < 1 || a->m > GDN_QLINEAR_MAX_ROWS || !gdn::qlinear_k_supported(a->k))
    return fail(GDN_EINVAL, "gdn_qlinear_workspace_size: bad shape (n_layers=%d m=%d k=%d)", a->n_layers, a->m, a->k);
  *bytes = gdn::qlinear_workspace_bytes(a->n_layers, a->m, a->k);
  return ok();
}

}  // extern "C"
