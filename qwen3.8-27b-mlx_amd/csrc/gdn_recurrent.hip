// Recurrent gated-delta kernel for gfx950: decode (T = 1), speculative verify
// (T steps, every per-step state written) and any other T.
//
// Work decomposition. One workgroup = 4 wave64s = one (layer, batch, v-head, Dv tile of
// 16 x SLOTS rows): 64 rows (SLOTS = 4, 32 KB of fp32 state) when the grid is large, 16
// rows (SLOTS = 1) when it is small -- a single-layer call, whose 96 tiles of 64 rows
// would leave most CUs idle. The state is read once and written once per call whatever
// T is. Each wave owns 4 x SLOTS state rows; inside a wave each 16-lane DPP row owns one
// state row at a time and a lane holds SLOTS rows ("slots") x 8 fp32 elements: [4j, 4j+4)
// and [64+4j, 64+4j+4) for lane j of the group, so one float4 load instruction of the
// wave reads 4 rows x 256 contiguous bytes. State traffic is non-temporal: it is streamed
// once per step and would only evict the small shared inputs from the caches.
//
// q, k, the tile's v rows and the gates of up to 8 steps are staged in LDS by the
// workgroup (computed there from x in the conv front end: causal depthwise conv,
// SiLU, l2norm, q scale, gate math) -- except in decode with q, k, v given, where each
// lane loads the 16 elements of q and k and the v values it uses itself -- then every
// wave applies the steps to its rows:
//   kS = k . s            (per-lane partial dot, then a 16-lane DPP butterfly)
//   s  = a (s - b kS k) + b v_r k
//   o_r = q . s           (partial dot + DPP butterfly)
// Both reductions stay inside a DPP row: no LDS, no atomics. For T > 1 with the conv front
// end each wave computes two steps of every pass of up to 8 (their q, k, v and gates); on
// 16-row tiles a block of more than 8 steps that records nothing runs on 8 waves instead,
// four of them computing the next pass's front end into a second LDS buffer while the
// other four apply the current pass's steps.
//
// Decode (T = 1) orders its memory traffic for latency: the front end's few loads are
// issued first, then the tile's state loads, so the front-end arithmetic runs while the
// state is in flight (loads retire in order, so the reverse order would make the front
// end wait for the whole tile).
//
// Workgroups are dispatched to the 8 XCDs round robin, and the workgroups that share a
// k-head (its v-heads x Dv tiles) read the same q/k inputs, so the block ids are renumbered
// to run them on one XCD, whose L2 then serves those reads after the first. Large grids
// (more than 16,384 workgroups: batched decode) give each XCD one contiguous eighth of the
// grid; smaller ones interleave: k-head group 8 s + x on XCD x, so the XCDs still stream
// neighbouring state. (The contiguous split measured slower for small grids, the
// interleaved one for B = 32: 1.84 against 1.64 ms.)
//
// Reference semantics: cpp/src/delta.cpp:185-200 (step), 87-94 (collect), the gates of
// cpp/src/model.cpp:608-612 and the front end of model.cpp:585-606 / 385-395.
#include "gdn_device_math.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

typedef float f4v __attribute__((ext_vector_type(4)));
typedef int i4v __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 waves
constexpr int kTC = 8;         // steps staged in LDS per pass

// Dv tile of 16 x SLOTS rows (SLOTS rows per 16-lane group, 4 groups per wave, 4 waves)
template <int SLOTS>
struct Geom {
  static constexpr int kSlots = SLOTS;
  static constexpr int kTileRows = 16 * SLOTS;
  static constexpr int kTilesPerHead = kD / kTileRows;
};
constexpr int kBigSlots = 4;    // 64-row tiles
constexpr int kSmallSlots = 1;  // 16-row tiles

// Butterfly sum over a whole wave64 in the fixed order p[l] += p[l ^ m],
// m = 1, 2, 4, 8, 16, 32: the l2norm sum order, fixed so that its bf16 rounding is
// reproducible (MLX does not pin the order of its bf16 reductions). m = 1..8 is the DPP
// row sum (bit for bit); after it row r holds its sum s_r on every lane, and the last two
// steps give every lane (s0 + s1) + (s2 + s3) (IEEE addition commutes), which is read
// off four lanes instead of a trip through the LDS crossbar per step (ds_bpermute): one
// layer's decode with the conv front end 4.11 -> 3.94 us, verify (B = 8, T = 5) 29.4 ->
// 28.5 us, together with the batched SiLU of the front ends.
__device__ __forceinline__ float wave64_sum(float x) {
  x = row16_sum(x);
  const float s0 = bits_f(__builtin_amdgcn_readlane(f_bits(x), 0));
  const float s1 = bits_f(__builtin_amdgcn_readlane(f_bits(x), 16));
  const float s2 = bits_f(__builtin_amdgcn_readlane(f_bits(x), 32));
  const float s3 = bits_f(__builtin_amdgcn_readlane(f_bits(x), 48));
  return (s0 + s1) + (s2 + s3);
}

// Causal depthwise conv at one channel from its 4 xp rows and 4 taps
// (model.cpp:385-395): taps in order j = 0..3, every product and partial sum rounded
// to bf16.
__device__ __forceinline__ float conv4(const float (&xv)[kTaps], const float (&wv)[kTaps]) {
  float y = rbf(xv[0] * wv[0]);
#pragma unroll
  for (int j = 1; j < kTaps; ++j) y = rbf(y + rbf(xv[j] * wv[j]));
  return y;
}

// l2norm of a 128-vector held as (u0, u1) = elements (lane, lane+64) of a wave
// (ops.cpp:27-30): x * rsqrt(sum(x*x) + eps), every op in bf16; q additionally gets the
// 128^-0.5 scale (model.cpp:601).
__device__ __forceinline__ void l2norm_pair(float u0, float u1, bool scale, float& y0, float& y1) {
  const float scale_b = rbf(1.0f / sqrtf((float)kD));
  const float eps_b = rbf(1e-6f);
  const float pr = rbf(u0 * u0) + rbf(u1 * u1);
  const float ssum = rbf(wave64_sum(pr));
  const float den = rbf(ssum + eps_b);
  const float rs = rsqrt_bf(den);
  y0 = rbf(u0 * rs);
  y1 = rbf(u1 * rs);
  if (scale) {
    y0 = rbf(y0 * scale_b);
    y1 = rbf(y1 * scale_b);
  }
}

struct Tile {
  int layer, bb, h, g, r0, tile;
  size_t lb, head;
};

// n / d, d one of the block map's divisors: with FAST as one scalar multiply-high by
// rc = ceil(2^32 / d) (0 for d = 1), exact since the host checked n d <= 2^32 for the grid;
// else the integer division (a sequence in the vector unit).
template <bool FAST>
__device__ __forceinline__ int map_div(int n, int d, uint32_t rc) {
  if constexpr (FAST) return rc ? (int)__umulhi((uint32_t)n, rc) : n;
  return n / d;
}

template <int SLOTS, bool FAST>
__device__ __forceinline__ Tile decode_block_as(const RecurrentParams& p) {
  int bid = blockIdx.x;
  const int gs = p.rep * Geom<SLOTS>::kTilesPerHead;  // workgroups of one k-head
  if (p.order == 1) {
    const int per = (int)gridDim.x >> 3;
    bid = (bid & 7) * per + (bid >> 3);
  } else if (p.order == 2) {
    // dispatch id d = 8 gs s + 8 j + x runs on XCD x as workgroup j of k-head group
    // 8 s + x: each k-head on one XCD, consecutive k-heads on consecutive XCDs
    const int s = map_div<FAST>(bid, 8 * gs, p.rc_grp8), r = bid - s * 8 * gs, j = r >> 3, x = r & 7;
    bid = gs * (8 * s + x) + j;
  }
  Tile t;
  t.tile = bid % Geom<SLOTS>::kTilesPerHead;
  const int rest = bid / Geom<SLOTS>::kTilesPerHead;
  const int lb = map_div<FAST>(rest, p.Hv, p.rc_hv);
  t.h = rest - lb * p.Hv;
  t.layer = map_div<FAST>(lb, p.B, p.rc_b);
  t.bb = lb - t.layer * p.B;
  t.g = map_div<FAST>(t.h, p.rep, p.rc_rep);
  t.r0 = t.tile * Geom<SLOTS>::kTileRows;
  t.lb = (size_t)t.layer * p.B + t.bb;
  t.head = t.lb * p.Hv + t.h;
  return t;
}

template <int SLOTS>
__device__ __forceinline__ Tile decode_block(const RecurrentParams& p) {
  return p.fastdiv ? decode_block_as<SLOTS, true>(p) : decode_block_as<SLOTS, false>(p);
}

template <int SLOTS>
__device__ __forceinline__ int row_of(int wave, int i, int grp) { return wave * 4 * SLOTS + i * 4 + grp; }

// The tile's rows of one (layer, batch, v-head) state at `base`.
template <int SLOTS>
__device__ __forceinline__ void load_rows(const float* base, const Tile& t, int wave, int grp, int j16,
                                          f4v (&s)[SLOTS][2]) {
#pragma unroll
  for (int i = 0; i < SLOTS; ++i) {
    const int row = t.r0 + row_of<SLOTS>(wave, i, grp);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      s[i][hf] = __builtin_nontemporal_load(
          reinterpret_cast<const f4v*>(base + (size_t)row * kD + hf * 64 + j16 * 4));
    }
  }
}

template <int SLOTS>
__device__ __forceinline__ void load_state(const RecurrentParams& p, const Tile& t, int wave,
                                           int grp, int j16, f4v (&s)[SLOTS][2]) {
  if (p.state_in) {
    load_rows<SLOTS>(p.state_in + t.head * kD * kD, t, wave, grp, j16, s);
  } else {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) s[i][0] = s[i][1] = f4v{0.f, 0.f, 0.f, 0.f};
  }
}

// State stores are non-temporal and written back. Writing the grid's last 40 MB through
// (device scope) instead, or every per-step state of a verify block, measured faster only
// while the benchmark's rotating state sets partly fitted the 256 MB last-level cache (4
// sets, 604 MB); with 8 sets (1.2 GB) it made the 48-layer B=1 step slower (53.7 -> 55.5
// us) and verify no faster, so every store writes back.
template <int SLOTS>
__device__ __forceinline__ void store_rows(float* base, const Tile& t, int wave, int grp, int j16,
                                           const f4v (&s)[SLOTS][2]) {
#pragma unroll
  for (int i = 0; i < SLOTS; ++i) {
    const int row = t.r0 + row_of<SLOTS>(wave, i, grp);
#pragma unroll
    for (int hf = 0; hf < 2; ++hf) {
      __builtin_nontemporal_store(s[i][hf],
                                  reinterpret_cast<f4v*>(base + (size_t)row * kD + hf * 64 + j16 * 4));
    }
  }
}

// The conv state hand-off: rows T..T+2 of [conv_in ; x] for this tile's v channels,
// plus the q (first tile) or k (second tile) channels of the k-head when h is its
// k-head's first v-head. Every channel has exactly one writer.
template <int SLOTS>
__device__ __forceinline__ void write_conv_out(const RecurrentParams& p, const Tile& t,
                                               const uint16_t* x_b, const uint16_t* cin_b) {
  constexpr int kTileRows = Geom<SLOTS>::kTileRows;
  uint16_t* cout_b = p.conv_out + t.lb * (size_t)kConvRows * p.C;
  const int vbase = 2 * p.Hk * kD + t.h * kD + t.r0;
  const bool qk_writer = t.h == t.g * p.rep && t.tile < 2;
  const int qkbase = (t.tile == 0 ? 0 : p.Hk * kD) + t.g * kD;
  const int nch = kTileRows + (qk_writer ? kD : 0);
  for (int e = threadIdx.x; e < nch * kConvRows; e += kThreads) {
    const int r = e / nch;
    const int ci = e % nch;
    const int c = ci < kTileRows ? vbase + ci : qkbase + (ci - kTileRows);
    const int src = p.T + r;  // row of xp
    uint16_t val;
    if (src < kConvRows) {
      val = cin_b ? cin_b[(size_t)src * p.C + c] : (uint16_t)0;
    } else {
      val = x_b[(size_t)(src - kConvRows) * p.C + c];
    }
    cout_b[(size_t)r * p.C + c] = val;
  }
}

// One step on the tile's rows in registers, from this lane's elements of k and q
// ([4 j16, 4 j16 + 4) and [64 + 4 j16, 64 + 4 j16 + 4)) and its slots' v values.
template <int SLOTS, bool COLLECT>
__device__ __forceinline__ void apply_step_r(const RecurrentParams& p, const Tile& t, int T, int step,
                                             float al, float be, f4v k0, f4v k1, f4v q0, f4v q1,
                                             const float (&vrs)[SLOTS], int wave, int grp, int j16,
                                             f4v (&s)[SLOTS][2]) {
  // with COLLECT, this step's state; each slot's rows go out as soon as they are updated
  float* const dst = !COLLECT ? nullptr
                     : p.states_tbh
                         ? p.states + ((((size_t)t.layer * T + step) * p.B + t.bb) * p.Hv + t.h) * kD * kD
                         : p.states + (t.head * T + step) * kD * kD;
  float ov[SLOTS];
#pragma unroll
  for (int i = 0; i < SLOTS; ++i) {
    const float vr = vrs[i];
    f4v& a0 = s[i][0];
    f4v& a1 = s[i][1];
    float pk = k0.x * a0.x;
    pk = __builtin_fmaf(k0.y, a0.y, pk);
    pk = __builtin_fmaf(k0.z, a0.z, pk);
    pk = __builtin_fmaf(k0.w, a0.w, pk);
    pk = __builtin_fmaf(k1.x, a1.x, pk);
    pk = __builtin_fmaf(k1.y, a1.y, pk);
    pk = __builtin_fmaf(k1.z, a1.z, pk);
    pk = __builtin_fmaf(k1.w, a1.w, pk);
    const float kS = row16_sum(pk);
    const float nbk = -(be * kS);
    const float bv = be * vr;
#define GDN_UPD(S, K) S = __builtin_fmaf(al, __builtin_fmaf(nbk, K, S), bv * K)
    GDN_UPD(a0.x, k0.x); GDN_UPD(a0.y, k0.y); GDN_UPD(a0.z, k0.z); GDN_UPD(a0.w, k0.w);
    GDN_UPD(a1.x, k1.x); GDN_UPD(a1.y, k1.y); GDN_UPD(a1.z, k1.z); GDN_UPD(a1.w, k1.w);
#undef GDN_UPD
    if (COLLECT) {
      const int row = t.r0 + row_of<SLOTS>(wave, i, grp);
      __builtin_nontemporal_store(a0, reinterpret_cast<f4v*>(dst + (size_t)row * kD + j16 * 4));
      __builtin_nontemporal_store(a1, reinterpret_cast<f4v*>(dst + (size_t)row * kD + 64 + j16 * 4));
    }
    float po = q0.x * a0.x;
    po = __builtin_fmaf(q0.y, a0.y, po);
    po = __builtin_fmaf(q0.z, a0.z, po);
    po = __builtin_fmaf(q0.w, a0.w, po);
    po = __builtin_fmaf(q1.x, a1.x, po);
    po = __builtin_fmaf(q1.y, a1.y, po);
    po = __builtin_fmaf(q1.z, a1.z, po);
    po = __builtin_fmaf(q1.w, a1.w, po);
    ov[i] = row16_sum(po);
  }

  // lane j (< SLOTS) of each group writes the output of slot j
  if (j16 < SLOTS) {
    float val = ov[0];
#pragma unroll
    for (int i = 1; i < SLOTS; ++i) val = (j16 == i) ? ov[i] : val;
    const int row = t.r0 + row_of<SLOTS>(wave, j16, grp);
    const size_t oi = ((t.lb * T + step) * p.Hv + t.h) * kD + row;
    if (p.o_bf16) {
      static_cast<uint16_t*>(p.o)[oi] = f2bf(val);
    } else {
      static_cast<float*>(p.o)[oi] = val;
    }
  }
}

// The same with k, q and the tile's v rows staged in LDS.
template <int SLOTS, bool COLLECT>
__device__ __forceinline__ void apply_step(const RecurrentParams& p, const Tile& t, int T, int step,
                                           float al, float be, const float* kk, const float* qq,
                                           const float* vv, int wave, int grp, int j16,
                                           f4v (&s)[SLOTS][2]) {
  const f4v k0 = *reinterpret_cast<const f4v*>(kk + j16 * 4);
  const f4v k1 = *reinterpret_cast<const f4v*>(kk + 64 + j16 * 4);
  const f4v q0 = *reinterpret_cast<const f4v*>(qq + j16 * 4);
  const f4v q1 = *reinterpret_cast<const f4v*>(qq + 64 + j16 * 4);
  float vrs[SLOTS];
#pragma unroll
  for (int i = 0; i < SLOTS; ++i) vrs[i] = vv[row_of<SLOTS>(wave, i, grp)];
  apply_step_r<SLOTS, COLLECT>(p, t, T, step, al, be, k0, k1, q0, q1, vrs, wave, grp, j16, s);
}

// Address of row r of the padded conv input xp = [conv_in ; x] at channel c. A row of a
// missing (zero) conv state points at x instead -- a valid address -- and its value is
// replaced by zero after the load (xp_value), so the loads carry no branches and can all
// be in flight together.
__device__ __forceinline__ const uint16_t* xp_addr(const uint16_t* __restrict__ x_b,
                                                   const uint16_t* __restrict__ cin_b, int C,
                                                   int c, int r) {
  if (r >= kConvRows) return x_b + (size_t)(r - kConvRows) * C + c;
  return cin_b ? cin_b + (size_t)r * C + c : x_b + c;
}

__device__ __forceinline__ float xp_value(uint32_t raw, const uint16_t* cin_b, int r) {
  return (r < kConvRows && !cin_b) ? 0.0f : bf2f((uint16_t)raw);
}

// Raw gate inputs of one (step, v-head): (a, b, A_log, dt_bias) or (alpha, beta).
struct GateRaw {
  uint32_t g0 = 0, g1 = 0, g2 = 0, g3 = 0;
};

__device__ __forceinline__ GateRaw gate_load(const RecurrentParams& p, int layer, int h, size_t gi) {
  GateRaw r;
  if (p.gate_raw) {
    r.g0 = p.a[gi];
    r.g1 = p.b[gi];
    r.g2 = f_bits(p.A_log[(size_t)layer * p.Hv + h]);
    r.g3 = f_bits(p.dt_bias[(size_t)layer * p.Hv + h]);
  } else {
    r.g0 = f_bits(p.alpha[gi]);
    r.g1 = f_bits(p.beta[gi]);
  }
  return r;
}

__device__ __forceinline__ void gate_math(const RecurrentParams& p, const GateRaw& r, float& al,
                                          float& be) {
  if (p.gate_raw) {
    d_gates(bf2f((uint16_t)r.g0), bf2f((uint16_t)r.g1), bits_f(r.g2), bits_f(r.g3), al, be);
  } else {
    al = bits_f(r.g0);
    be = bits_f(r.g1);
  }
}

__device__ __forceinline__ uint32_t qkv_raw(const void* base, size_t i, int bf16) {
  return bf16 ? (uint32_t) static_cast<const uint16_t*>(base)[i]
              : static_cast<const uint32_t*>(base)[i];
}

__device__ __forceinline__ float qkv_value(uint32_t raw, int bf16) {
  return bf16 ? bf2f((uint16_t)raw) : bits_f(raw);
}

// Front-end channel of a wave in the conv front end: wave 0 -> q channels (lane,
// lane+64) of k-head g, wave 1 -> k channels, wave 2 -> the tile's v channels (lanes past
// the tile's rows repeat its last channel: their values go unused).
template <int SLOTS>
__device__ __forceinline__ int fe_channel(const RecurrentParams& p, const Tile& t, int wave,
                                          int lane) {
  return wave == 0 ? t.g * kD + lane
       : wave == 1 ? p.Hk * kD + t.g * kD + lane
                   : 2 * p.Hk * kD + t.h * kD + t.r0 + min(lane, Geom<SLOTS>::kTileRows - 1);
}

// ---------------------------------------------------------------- decode, T = 1

// q, k, v given (the reference's delta::run inputs): every lane loads its own elements of
// q and k and its slots' v values, and every wave does the gate math, so there is no LDS
// staging and no barrier; with the state present there is no branch around any load, so
// nothing but the step itself waits for the state. VEC: q and k aligned to 4 elements, read
// 4 elements per load (else one element per load).
template <int SLOTS, bool HAS_STATE, bool VEC>
__global__ __launch_bounds__(kThreads) void decode_qkv_kernel(RecurrentParams p) {
  typedef int i2v __attribute__((ext_vector_type(2)));
  const Tile t = decode_block<SLOTS>(p);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int grp = lane >> 4, j16 = lane & 15;
  const size_t row0 = t.lb;  // (layer, b) at step 0

  // 1. loads: q and k raw (bf16 pairs or fp32), v of the slots' rows, gates, the state
  i4v qr[2], kr[2];
  const size_t qkb = (row0 * p.Hk + t.g) * kD + 4 * j16;
  if constexpr (!VEC) {
    // element by element, packed as the vector loads would leave them
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      uint32_t qe[4], ke[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qe[e] = qkv_raw(p.q, qkb + 64 * h2 + e, p.qkv_bf16);
        ke[e] = qkv_raw(p.k, qkb + 64 * h2 + e, p.qkv_bf16);
      }
      qr[h2] = p.qkv_bf16 ? i4v{(int)(qe[0] | qe[1] << 16), (int)(qe[2] | qe[3] << 16), 0, 0}
                          : i4v{(int)qe[0], (int)qe[1], (int)qe[2], (int)qe[3]};
      kr[h2] = p.qkv_bf16 ? i4v{(int)(ke[0] | ke[1] << 16), (int)(ke[2] | ke[3] << 16), 0, 0}
                          : i4v{(int)ke[0], (int)ke[1], (int)ke[2], (int)ke[3]};
    }
  } else if (p.qkv_bf16) {
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const i2v a = *reinterpret_cast<const i2v*>(static_cast<const uint16_t*>(p.q) + qkb + 64 * h2);
      const i2v b = *reinterpret_cast<const i2v*>(static_cast<const uint16_t*>(p.k) + qkb + 64 * h2);
      qr[h2] = i4v{a.x, a.y, 0, 0};
      kr[h2] = i4v{b.x, b.y, 0, 0};
    }
  } else {
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      qr[h2] = *reinterpret_cast<const i4v*>(static_cast<const float*>(p.q) + qkb + 64 * h2);
      kr[h2] = *reinterpret_cast<const i4v*>(static_cast<const float*>(p.k) + qkb + 64 * h2);
    }
  }
  uint32_t vraw[SLOTS];
#pragma unroll
  for (int i = 0; i < SLOTS; ++i)
    vraw[i] = qkv_raw(p.v, (row0 * p.Hv + t.h) * kD + t.r0 + row_of<SLOTS>(wave, i, grp), p.qkv_bf16);
  const GateRaw gr = gate_load(p, t.layer, t.h, row0 * p.Hv + t.h);
  f4v s[SLOTS][2];
  if constexpr (HAS_STATE) {
    load_rows<SLOTS>(p.state_in + t.head * kD * kD, t, wave, grp, j16, s);
  } else {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) s[i][0] = s[i][1] = f4v{0.f, 0.f, 0.f, 0.f};
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the arithmetic below the loads

  // 2. gates and values while the state is in flight, then the step
  float al, be;
  gate_math(p, gr, al, be);
  f4v qf[2], kf[2];
#pragma unroll
  for (int h2 = 0; h2 < 2; ++h2) {
    if (p.qkv_bf16) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        qf[h2][e] = bf2f((uint16_t)((uint32_t)qr[h2][e >> 1] >> (16 * (e & 1))));
        kf[h2][e] = bf2f((uint16_t)((uint32_t)kr[h2][e >> 1] >> (16 * (e & 1))));
      }
    } else {
      qf[h2] = __builtin_bit_cast(f4v, qr[h2]);
      kf[h2] = __builtin_bit_cast(f4v, kr[h2]);
    }
  }
  float vrs[SLOTS];
#pragma unroll
  for (int i = 0; i < SLOTS; ++i) vrs[i] = qkv_value(vraw[i], p.qkv_bf16);
  apply_step_r<SLOTS, false>(p, t, 1, 0, al, be, kf[0], kf[1], qf[0], qf[1], vrs, wave, grp, j16, s);
  if (p.state_out) store_rows<SLOTS>(p.state_out + t.head * kD * kD, t, wave, grp, j16, s);
}

// The conv front end (x and the conv state given): q, k, v computed in the workgroup and
// staged in LDS.
template <int SLOTS>
__global__ __launch_bounds__(kThreads) void decode_kernel(RecurrentParams p) {
  constexpr int kTileRows = Geom<SLOTS>::kTileRows;
  __shared__ float sm_q[kD];
  __shared__ float sm_k[kD];
  __shared__ float sm_v[kTileRows];
  __shared__ float sm_ab[2];

  const Tile t = decode_block<SLOTS>(p);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = lane >> 4, j16 = lane & 15;
  const size_t row0 = t.lb;  // (layer, b) at step 0

  // 1. the front end's global loads, all in flight together
  uint32_t xr[2][kTaps], wr[2][kTaps];
  const uint16_t* x_b = p.x + t.lb * (size_t)p.C;
  const uint16_t* cin_b = p.conv_in ? p.conv_in + t.lb * (size_t)kConvRows * p.C : nullptr;
  int c0 = 0;
  {
    const uint16_t* w_l = p.conv_w + (size_t)t.layer * kTaps * p.C;
    // Every wave issues the same loads (no branch, so nothing waits on them early);
    // waves 2 and 3 read their one channel twice, wave 3's values go unused.
    c0 = fe_channel<SLOTS>(p, t, wave < 3 ? wave : 2, lane);
    const int c1 = wave < 2 ? c0 + 64 : c0;
#pragma unroll
    for (int j = 0; j < kTaps; ++j) {
      xr[0][j] = *xp_addr(x_b, cin_b, p.C, c0, j);
      wr[0][j] = w_l[(size_t)j * p.C + c0];
      xr[1][j] = *xp_addr(x_b, cin_b, p.C, c1, j);
      wr[1][j] = w_l[(size_t)j * p.C + c1];
    }
  }
  // 2. the tile's state; then the gate inputs, which only wave 3 waits for
  f4v s[SLOTS][2];
  load_state<SLOTS>(p, t, wave, grp, j16, s);
  GateRaw gr;
  if (wave == 3) gr = gate_load(p, t.layer, t.h, row0 * p.Hv + t.h);
  __builtin_amdgcn_sched_barrier(0);  // keep the front-end arithmetic below the loads

  // 3. front-end arithmetic while the state is in flight
  if (wave < 3) {
    float u[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      float xv[kTaps], wv[kTaps];
#pragma unroll
      for (int j = 0; j < kTaps; ++j) {
        xv[j] = xp_value(xr[m][j], cin_b, j);
        wv[j] = bf2f((uint16_t)wr[m][j]);
      }
      u[m] = conv4(xv, wv);
    }
    silu_bf_batch(u);
    if (wave < 2) {
      float y0, y1;
      l2norm_pair(u[0], u[1], wave == 0, y0, y1);
      float* dst = wave == 0 ? sm_q : sm_k;
      dst[lane] = y0;
      dst[lane + 64] = y1;
    } else if (lane < kTileRows) {
      sm_v[lane] = u[0];
    }
  }
  if (wave == 3) {
    float al, be;
    gate_math(p, gr, al, be);
    if (lane == 0) {
      sm_ab[0] = al;
      sm_ab[1] = be;
    }
  }
  __syncthreads();

  // 4. the step, then the state goes back
  apply_step<SLOTS, false>(p, t, 1, 0, sm_ab[0], sm_ab[1], sm_k, sm_q, sm_v, wave, grp, j16, s);
  if (p.state_out) store_rows<SLOTS>(p.state_out + t.head * kD * kD, t, wave, grp, j16, s);

  // 5. conv state hand-off from the rows already in registers: new rows 0..2 are xp
  // rows 1..3. This tile's v channels; the q (tile 0) or k (tile 1) channels of the
  // k-head when h is its k-head's first v-head -- every channel has one writer.
  if (p.conv_out) {
    uint16_t* cout_b = p.conv_out + t.lb * (size_t)kConvRows * p.C;
    const bool qk_writer = t.h == t.g * p.rep && wave == t.tile;
    const int nm = wave == 2 ? (lane < kTileRows ? 1 : 0) : (wave < 2 && qk_writer ? 2 : 0);
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      if (m < nm) {
#pragma unroll
        for (int r = 0; r < kConvRows; ++r) {
          const bool zero = (r + 1 < kConvRows) && !cin_b;
          cout_b[(size_t)r * p.C + c0 + 64 * m] = zero ? (uint16_t)0 : (uint16_t)xr[m][r + 1];
        }
      }
    }
  }
}

// ---------------------------------------------------------------- any T (verify, prefill-size L)

template <bool B>
struct BoolTag {
  static constexpr bool value = B;
};

// Every load of a pass is issued unconditionally (addresses clamped to valid rows, values
// past the pass unused) and the first pass, which also loads the state, is a separate
// instantiation of the pass: a load under a data-dependent branch would make the compiler
// count the loads after it conservatively at the join, so the front end would wait for the
// whole state tile (or each conv row for the previous one) before its arithmetic.
template <int SLOTS, int FE, bool COLLECT, bool HAS_STATE>
__global__ __launch_bounds__(kThreads) void steps_kernel(RecurrentParams p) {
  constexpr int kTileRows = Geom<SLOTS>::kTileRows;
  __shared__ float sm_q[kTC][kD];
  __shared__ float sm_k[kTC][kD];
  __shared__ float sm_v[kTC][kTileRows];
  __shared__ float sm_a[kTC];
  __shared__ float sm_b[kTC];

  const Tile t = decode_block<SLOTS>(p);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int grp = lane >> 4, j16 = lane & 15;
  const int T = p.T;
  constexpr int kPer = 2 * kD + kTileRows;  // q, k, v values of one step (FE = 0)
  constexpr int kRaw = (kTC * kPer + kThreads - 1) / kThreads;

  const uint16_t* x_b = nullptr;
  const uint16_t* cin_b = nullptr;
  // conv front end: wave w takes steps 2 w and 2 w + 1 of every pass, all of their q, k and
  // v channels -- lane l: q and k channels (l, l + 64) of the k-head and the tile's v row l
  // (lanes past the tile's rows repeat its last one; their values go unused)
  constexpr int kFeCh = 5, kFeRows = 2 + kTaps - 1;
  int ch[kFeCh] = {};
  float wv[kFeCh][kTaps] = {};
  if (FE == 1) {
    x_b = p.x + t.lb * (size_t)T * p.C;
    cin_b = p.conv_in ? p.conv_in + t.lb * (size_t)kConvRows * p.C : nullptr;
    const uint16_t* w_l = p.conv_w + (size_t)t.layer * kTaps * p.C;
    ch[0] = fe_channel<SLOTS>(p, t, 0, lane);
    ch[1] = ch[0] + 64;
    ch[2] = fe_channel<SLOTS>(p, t, 1, lane);
    ch[3] = ch[2] + 64;
    ch[4] = fe_channel<SLOTS>(p, t, 2, lane);
#pragma unroll
    for (int c = 0; c < kFeCh; ++c) {
#pragma unroll
      for (int j = 0; j < kTaps; ++j) wv[c][j] = bf2f(w_l[(size_t)j * p.C + ch[c]]);
    }
  }
  // gates: lanes 0 and 1 of wave w for steps 2 w and 2 w + 1 (FE = 1); else the last 8
  // threads, one step each
  const int gt = FE == 1 ? (lane < 2 ? 2 * wave + lane : -1) : tid - (kThreads - kTC);
  const int gload = FE == 1 ? 2 * wave + (lane & 1) : gt;  // the step whose gates a thread loads

  f4v s[SLOTS][2];
  auto pass = [&](int t0, auto first) {
    constexpr bool kFirst = decltype(first)::value;
    const int tc = min(kTC, T - t0);
    if (!kFirst) __syncthreads();  // the previous pass is done reading LDS

    // 1. loads: the pass's conv window or q/k/v, its gates, and (first pass) the state
    uint32_t xr[kFeCh][kFeRows] = {};
    uint32_t raw[kRaw] = {};
    if (FE == 1) {
      const int last = T + kConvRows - 1;  // last row of xp = [conv_in ; x]
#pragma unroll
      for (int r = 0; r < kFeRows; ++r) {
        const int rr = min(t0 + 2 * wave + r, last);
#pragma unroll
        for (int c = 0; c < kFeCh; ++c) xr[c][r] = *xp_addr(x_b, cin_b, p.C, ch[c], rr);
      }
    } else {
#pragma unroll
      for (int i = 0; i < kRaw; ++i) {
        const int e = min(tid + i * kThreads, tc * kPer - 1);
        const int tt = e / kPer, c = e % kPer;
        const size_t row = t.lb * T + (t0 + tt);
        const void* base = c < kD ? p.q : c < 2 * kD ? p.k : p.v;
        const size_t idx = c < 2 * kD ? (row * p.Hk + t.g) * kD + (c & (kD - 1))
                                      : (row * p.Hv + t.h) * kD + t.r0 + (c - 2 * kD);
        raw[i] = qkv_raw(base, idx, p.qkv_bf16);
      }
    }
    const int gsel = min(max(gload, 0), tc - 1);
    const GateRaw gr = gate_load(p, t.layer, t.h, (t.lb * T + (t0 + gsel)) * p.Hv + t.h);
    if constexpr (kFirst) {
      if constexpr (HAS_STATE) {
        load_rows<SLOTS>(p.state_in + t.head * kD * kD, t, wave, grp, j16, s);
      } else {
#pragma unroll
        for (int i = 0; i < SLOTS; ++i) s[i][0] = s[i][1] = f4v{0.f, 0.f, 0.f, 0.f};
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the arithmetic below the loads

    // 2. front end into LDS while the state is in flight
    if (FE == 0) {
#pragma unroll
      for (int i = 0; i < kRaw; ++i) {
        const int e = tid + i * kThreads;
        if (e < tc * kPer) {
          const int tt = e / kPer, c = e % kPer;
          const float val = qkv_value(raw[i], p.qkv_bf16);
          if (c < kD) sm_q[tt][c] = val;
          else if (c < 2 * kD) sm_k[tt][c - kD] = val;
          else sm_v[tt][c - 2 * kD] = val;
        }
      }
    } else {
#pragma unroll
      for (int k2 = 0; k2 < 2; ++k2) {
        const int tt = 2 * wave + k2;
        if (tt < tc) {
          float u[kFeCh + 1];
#pragma unroll
          for (int c = 0; c < kFeCh; ++c) {
            float xv[kTaps];
#pragma unroll
            for (int j = 0; j < kTaps; ++j) xv[j] = xp_value(xr[c][k2 + j], cin_b, t0 + tt + j);
            u[c] = conv4(xv, wv[c]);
          }
          u[kFeCh] = 0.0f;
          silu_bf_batch(u);
          float y0, y1;
          l2norm_pair(u[0], u[1], true, y0, y1);
          sm_q[tt][lane] = y0;
          sm_q[tt][lane + 64] = y1;
          l2norm_pair(u[2], u[3], false, y0, y1);
          sm_k[tt][lane] = y0;
          sm_k[tt][lane + 64] = y1;
          if (lane < kTileRows) sm_v[tt][lane] = u[4];
        }
      }
    }
    if (gt >= 0 && gt < tc) gate_math(p, gr, sm_a[gt], sm_b[gt]);
    __syncthreads();

    // 3. the pass's steps on the rows in registers
    for (int tt = 0; tt < tc; ++tt) {
      apply_step<SLOTS, COLLECT>(p, t, T, t0 + tt, sm_a[tt], sm_b[tt], sm_k[tt], sm_q[tt], sm_v[tt], wave, grp,
                                 j16, s);
    }
  };
  pass(0, BoolTag<true>{});
  for (int t0 = kTC; t0 < T; t0 += kTC) pass(t0, BoolTag<false>{});

  if (p.state_out) store_rows<SLOTS>(p.state_out + t.head * kD * kD, t, wave, grp, j16, s);
  if (FE == 1 && p.conv_out) write_conv_out<SLOTS>(p, t, x_b, cin_b);
}

// Any T > 8 without per-step states, conv front end, 16-row tiles: 8 waves. Waves 0..3 hold the tile's
// state rows and run the steps of pass p from one LDS buffer while waves 4..7 compute the
// conv front end of pass p + 1 into the other (wave 4 + w: steps 2 w and 2 w + 1 of the pass,
// their q, k and v channels and their gates, as in steps_kernel); one barrier per pass, the
// same count in every wave. On a SIMD the front-end wave's independent work fills the issue
// slots that the steps' dependent chains leave idle.
template <int SLOTS, bool HAS_STATE>
__global__ __launch_bounds__(2 * kThreads) void steps_overlap_kernel(RecurrentParams p) {
  constexpr int kTileRows = Geom<SLOTS>::kTileRows;
  __shared__ float sm_q[2][kTC][kD];
  __shared__ float sm_k[2][kTC][kD];
  __shared__ float sm_v[2][kTC][kTileRows];
  __shared__ float sm_a[2][kTC];
  __shared__ float sm_b[2][kTC];

  const Tile t = decode_block<SLOTS>(p);
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool fe_wave = wave >= 4;
  const int fw = wave & 3;
  const int grp = lane >> 4, j16 = lane & 15;
  const int T = p.T;
  const uint16_t* x_b = p.x + t.lb * (size_t)T * p.C;
  const uint16_t* cin_b = p.conv_in ? p.conv_in + t.lb * (size_t)kConvRows * p.C : nullptr;
  constexpr int kFeCh = 5, kFeRows = 2 + kTaps - 1;
  int ch[kFeCh] = {};
  float wv[kFeCh][kTaps] = {};

  // the front end of the pass at t0 into buffer buf (front-end waves)
  auto fe_pass = [&](int t0, int buf) {
    const int tc = min(kTC, T - t0);
    uint32_t xr[kFeCh][kFeRows];
    const int last = T + kConvRows - 1;  // last row of xp = [conv_in ; x]
#pragma unroll
    for (int r = 0; r < kFeRows; ++r) {
      const int rr = min(t0 + 2 * fw + r, last);
#pragma unroll
      for (int c = 0; c < kFeCh; ++c) xr[c][r] = *xp_addr(x_b, cin_b, p.C, ch[c], rr);
    }
    const int gsel = min(2 * fw + (lane & 1), tc - 1);
    const GateRaw gr = gate_load(p, t.layer, t.h, (t.lb * T + (t0 + gsel)) * p.Hv + t.h);
#pragma unroll
    for (int k2 = 0; k2 < 2; ++k2) {
      const int tt = 2 * fw + k2;
      if (tt < tc) {
        float u[kFeCh + 1];
#pragma unroll
        for (int c = 0; c < kFeCh; ++c) {
          float xv[kTaps];
#pragma unroll
          for (int j = 0; j < kTaps; ++j) xv[j] = xp_value(xr[c][k2 + j], cin_b, t0 + tt + j);
          u[c] = conv4(xv, wv[c]);
        }
        u[kFeCh] = 0.0f;
        silu_bf_batch(u);
        float y0, y1;
        l2norm_pair(u[0], u[1], true, y0, y1);
        sm_q[buf][tt][lane] = y0;
        sm_q[buf][tt][lane + 64] = y1;
        l2norm_pair(u[2], u[3], false, y0, y1);
        sm_k[buf][tt][lane] = y0;
        sm_k[buf][tt][lane + 64] = y1;
        if (lane < kTileRows) sm_v[buf][tt][lane] = u[4];
      }
    }
    const int gt = 2 * fw + lane;
    if (lane < 2 && gt < tc) gate_math(p, gr, sm_a[buf][gt], sm_b[buf][gt]);
  };

  f4v s[SLOTS][2];
  if (fe_wave) {
    const uint16_t* w_l = p.conv_w + (size_t)t.layer * kTaps * p.C;
    ch[0] = fe_channel<SLOTS>(p, t, 0, lane);
    ch[1] = ch[0] + 64;
    ch[2] = fe_channel<SLOTS>(p, t, 1, lane);
    ch[3] = ch[2] + 64;
    ch[4] = fe_channel<SLOTS>(p, t, 2, lane);
#pragma unroll
    for (int c = 0; c < kFeCh; ++c) {
#pragma unroll
      for (int j = 0; j < kTaps; ++j) wv[c][j] = bf2f(w_l[(size_t)j * p.C + ch[c]]);
    }
    fe_pass(0, 0);
  } else if constexpr (HAS_STATE) {
    load_rows<SLOTS>(p.state_in + t.head * kD * kD, t, wave, grp, j16, s);
  } else {
#pragma unroll
    for (int i = 0; i < SLOTS; ++i) s[i][0] = s[i][1] = f4v{0.f, 0.f, 0.f, 0.f};
  }
  __syncthreads();  // pass 0's front end is in buffer 0

  int buf = 0;
  for (int t0 = 0; t0 < T; t0 += kTC) {
    if (fe_wave) {
      if (t0 + kTC < T) fe_pass(t0 + kTC, buf ^ 1);
    } else {
      const int tc = min(kTC, T - t0);
      for (int tt = 0; tt < tc; ++tt) {
        apply_step<SLOTS, false>(p, t, T, t0 + tt, sm_a[buf][tt], sm_b[buf][tt], sm_k[buf][tt], sm_q[buf][tt],
                                 sm_v[buf][tt], wave, grp, j16, s);
      }
    }
    __syncthreads();  // buffer buf is read, buffer buf ^ 1 is written
    buf ^= 1;
  }

  if (!fe_wave) {
    if (p.state_out) store_rows<SLOTS>(p.state_out + t.head * kD * kD, t, wave, grp, j16, s);
    if (p.conv_out) write_conv_out<SLOTS>(p, t, x_b, cin_b);
  }
}

__global__ void copy_f32_kernel(float* __restrict__ dst, const float* __restrict__ src, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    dst[i] = src ? src[i] : 0.0f;
  }
}

__global__ void copy_u16_kernel(uint16_t* __restrict__ dst, const uint16_t* __restrict__ src,
                                int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    dst[i] = src ? src[i] : (uint16_t)0;
  }
}

// The 16-row tiles serve grids whose 64-row form would be small: up to this many
// (layer, batch, v-head) units, i.e. at most 2 x kSmallTileMaxHeads 64-row workgroups.
#ifndef GDN_SMALL_TILE_MAX_HEADS
#define GDN_SMALL_TILE_MAX_HEADS 96
#endif
constexpr long long kSmallTileMaxHeads = GDN_SMALL_TILE_MAX_HEADS;

template <int SLOTS, int FE, bool HAS_STATE>
void launch_steps_s(const RecurrentParams& p, bool collect, dim3 grid, dim3 block, hipStream_t stream) {
  if (collect) hipLaunchKernelGGL((steps_kernel<SLOTS, FE, true, HAS_STATE>), grid, block, 0, stream, p);
  else hipLaunchKernelGGL((steps_kernel<SLOTS, FE, false, HAS_STATE>), grid, block, 0, stream, p);
}

template <int SLOTS, int FE>
void launch_steps(const RecurrentParams& p, bool collect, dim3 grid, dim3 block, hipStream_t stream) {
  if (p.state_in) launch_steps_s<SLOTS, FE, true>(p, collect, grid, block, stream);
  else launch_steps_s<SLOTS, FE, false>(p, collect, grid, block, stream);
}

template <int SLOTS>
void launch_slots(const RecurrentParams& p, int frontend, bool collect, hipStream_t stream) {
  const dim3 grid(p.nblocks), block(kThreads);
  if (p.T == 1 && !collect) {
    const uintptr_t vec = p.qkv_bf16 ? 8 : 16;  // 4 elements
    const bool aligned = (reinterpret_cast<uintptr_t>(p.q) | reinterpret_cast<uintptr_t>(p.k)) % vec == 0;
    if (frontend == 1) hipLaunchKernelGGL((decode_kernel<SLOTS>), grid, block, 0, stream, p);
    else if (p.state_in && aligned) hipLaunchKernelGGL((decode_qkv_kernel<SLOTS, true, true>), grid, block, 0, stream, p);
    else if (p.state_in) hipLaunchKernelGGL((decode_qkv_kernel<SLOTS, true, false>), grid, block, 0, stream, p);
    else if (aligned) hipLaunchKernelGGL((decode_qkv_kernel<SLOTS, false, true>), grid, block, 0, stream, p);
    else hipLaunchKernelGGL((decode_qkv_kernel<SLOTS, false, false>), grid, block, 0, stream, p);
  } else if (frontend == 0) {
    launch_steps<SLOTS, 0>(p, collect, grid, block, stream);
  } else if (SLOTS == kSmallSlots && !collect && p.T > kTC) {
    // several passes on small grids: the front end of each pass overlaps the previous steps
    // (on 64-row tiles the 8-wave workgroups' registers leave one per CU: slower there)
    if constexpr (SLOTS == kSmallSlots) {
      const dim3 block2(2 * kThreads);
      if (p.state_in) hipLaunchKernelGGL((steps_overlap_kernel<SLOTS, true>), grid, block2, 0, stream, p);
      else hipLaunchKernelGGL((steps_overlap_kernel<SLOTS, false>), grid, block2, 0, stream, p);
    }
  } else {
    launch_steps<SLOTS, 1>(p, collect, grid, block, stream);
  }
}

}  // namespace

int recurrent_tile_rows(long long heads) {
  return heads <= kSmallTileMaxHeads ? Geom<kSmallSlots>::kTileRows : Geom<kBigSlots>::kTileRows;
}

hipError_t launch_recurrent(const RecurrentParams& p, int frontend, bool collect,
                            hipStream_t stream) {
  const long long heads = (long long)p.n_layers * p.B * p.Hv;
  if (recurrent_tile_rows(heads) == Geom<kSmallSlots>::kTileRows) launch_slots<kSmallSlots>(p, frontend, collect, stream);
  else launch_slots<kBigSlots>(p, frontend, collect, stream);
  return hipGetLastError();
}

hipError_t launch_copy_f32(float* dst, const float* src, int64_t n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(copy_f32_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, dst, src, n);
  return hipGetLastError();
}

hipError_t launch_copy_u16(uint16_t* dst, const uint16_t* src, int64_t n, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(copy_u16_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, dst, src, n);
  return hipGetLastError();
}

}  // namespace gdn
