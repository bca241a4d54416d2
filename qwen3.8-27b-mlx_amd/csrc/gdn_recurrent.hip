// Recurrent gated-delta kernel for gfx950: decode (T = 1), speculative verify
// (T steps, every per-step state written) and any other T.
//
// Work decomposition. One workgroup = 4 wave64s = one (layer, batch, v-head,
// 64-row Dv tile). Each wave owns 16 state rows; inside a wave, each 16-lane row of
// the wave (a DPP row) owns one state row at a time and the wave holds 4 rows per
// lane group ("slots"), so a lane keeps 4 x 8 fp32 state elements in registers.
// Lane j of a group holds elements [4j, 4j+4) and [64+4j, 64+4j+4) of its rows: one
// float4 load instruction of the wave reads 4 rows x 256 contiguous bytes.
//
// The state is read once and written once per call whatever T is: rows stay in
// registers while the steps run. q, k, v and the gates of up to 8 steps are staged
// in LDS by the workgroup (computed there from x in the conv front end), then every
// wave applies the steps to its rows:
//   kS = k . s            (per-lane partial dot, then a 16-lane DPP butterfly)
//   s  = a (s - b kS k) + b v_r k
//   o_r = q . s           (partial dot + DPP butterfly)
// Both reductions stay inside a DPP row: no LDS, no atomics.
//
// Reference semantics: cpp/src/delta.cpp:185-200 (step), 87-94 (collect), the gates
// of cpp/src/model.cpp:608-612 and the front end of model.cpp:585-606 / 385-395.
#include "gdn_device_math.h"
#include "gdn_internal.h"

namespace gdn {
namespace {

constexpr int kTileRows = 64;   // Dv rows per workgroup
constexpr int kThreads = 256;   // 4 waves
constexpr int kSlots = 4;       // rows per 16-lane group
constexpr int kTC = 8;          // steps staged in LDS per pass

// Sum over the 16 lanes of a DPP row; every lane receives the same total.
// quad_perm[1,0,3,2], quad_perm[2,3,0,1], row_half_mirror, row_mirror.
__device__ __forceinline__ float row16_sum(float x) {
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0xB1, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x4E, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x141, 0xF, 0xF, true));
  x += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, x), 0x140, 0xF, 0xF, true));
  return x;
}

// Butterfly sum over a whole wave64 in the fixed order p[l] += p[l ^ m],
// m = 1, 2, 4, 8, 16, 32: the l2norm sum order, fixed so that its bf16 rounding is
// reproducible (MLX does not pin the order of its bf16 reductions).
__device__ __forceinline__ float wave64_sum(float x) {
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) x = x + __shfl_xor(x, m, 64);
  return x;
}

__device__ __forceinline__ float load_qkv(const void* base, size_t i, int bf16) {
  return bf16 ? bf2f(static_cast<const uint16_t*>(base)[i]) : static_cast<const float*>(base)[i];
}

// One conv channel at step t (model.cpp:385-395): taps in order j = 0..3, every
// product and partial sum rounded to bf16; xp row r is conv_in[r] for r < 3 else x[r-3].
__device__ __forceinline__ float conv_channel(const uint16_t* __restrict__ x_b,
                                              const uint16_t* __restrict__ cin_b,
                                              const uint16_t* __restrict__ w, int C, int c,
                                              int t) {
  float y = 0.0f;
#pragma unroll
  for (int j = 0; j < kTaps; ++j) {
    const int r = t + j;
    float xv;
    if (r < kConvRows) {
      xv = cin_b ? bf2f(cin_b[(size_t)r * C + c]) : 0.0f;
    } else {
      xv = bf2f(x_b[(size_t)(r - kConvRows) * C + c]);
    }
    const float prod = rbf(xv * bf2f(w[(size_t)j * C + c]));
    y = (j == 0) ? prod : rbf(y + prod);
  }
  return y;
}

// silu on a bf16 value: x * sigmoid(x), both ops rounded (ops.cpp:20).
__device__ __forceinline__ float silu_bf(float y) {
  const float sg = rbf(d_sigmoidf(y));
  return rbf(y * sg);
}

template <int FE, bool COLLECT>
__global__ __launch_bounds__(kThreads) void recurrent_kernel(RecurrentParams p) {
  __shared__ float4 sm_q[kTC][kD / 4];
  __shared__ float4 sm_k[kTC][kD / 4];
  __shared__ float sm_v[kTC][kTileRows];
  __shared__ float sm_a[kTC];
  __shared__ float sm_b[kTC];

  int bid = blockIdx.x;
  if (p.remap) {
    // Consecutive logical blocks (the 3 v-heads x 2 tiles that share a k-head) land on
    // the same XCD, whose L2 then serves their shared q/k/x reads.
    const int per = p.nblocks >> 3;
    bid = (bid & 7) * per + (bid >> 3);
  }
  const int tile = bid & 1;
  int rest = bid >> 1;
  const int h = rest % p.Hv;
  rest /= p.Hv;
  const int bb = rest % p.B;
  const int layer = rest / p.B;
  const int g = h / p.rep;
  const int r0 = tile * kTileRows;

  const int tid = threadIdx.x;
  const int wave = tid >> 6;
  const int lane = tid & 63;
  const int grp = lane >> 4;
  const int j16 = lane & 15;

  const int T = p.T;
  const size_t lb = (size_t)layer * p.B + bb;         // (layer, b)
  const size_t head = lb * p.Hv + h;                  // (layer, b, h)
  const size_t DD = (size_t)kD * kD;

  // ---- issue the state loads first: they do not depend on the front end ----
  float4 s[kSlots][2];
  {
    const float* sin = p.state_in ? p.state_in + head * DD : nullptr;
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int row = r0 + wave * 16 + i * 4 + grp;
#pragma unroll
      for (int hf = 0; hf < 2; ++hf) {
        if (sin) {
          s[i][hf] = *reinterpret_cast<const float4*>(sin + (size_t)row * kD + hf * 64 + j16 * 4);
        } else {
          s[i][hf] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
      }
    }
  }

  // ---- conv state hand-off (conv front end): rows T..T+2 of [conv_in ; x] ----
  const uint16_t* x_b = nullptr;
  const uint16_t* cin_b = nullptr;
  const uint16_t* w_l = nullptr;
  if (FE == 1) {
    x_b = p.x + lb * (size_t)T * p.C;
    cin_b = p.conv_in ? p.conv_in + lb * (size_t)kConvRows * p.C : nullptr;
    w_l = p.conv_w + (size_t)layer * kTaps * p.C;
    if (p.conv_out) {
      uint16_t* cout_b = p.conv_out + lb * (size_t)kConvRows * p.C;
      // v channels of this tile; q (tile 0) or k (tile 1) channels of the k-head when
      // this is the k-head's first v-head. Each channel has exactly one writer.
      const int vbase = 2 * p.Hk * kD + h * kD + r0;
      const bool qk_writer = (h % p.rep) == 0;
      const int qkbase = (tile == 0 ? 0 : p.Hk * kD) + g * kD;
      const int nch = kTileRows + (qk_writer ? kD : 0);
      for (int e = tid; e < nch * kConvRows; e += kThreads) {
        const int r = e / nch;
        const int ci = e % nch;
        const int c = ci < kTileRows ? vbase + ci : qkbase + (ci - kTileRows);
        const int src = T + r;  // row of xp
        uint16_t val;
        if (src < kConvRows) {
          val = cin_b ? cin_b[(size_t)src * p.C + c] : (uint16_t)0;
        } else {
          val = x_b[(size_t)(src - kConvRows) * p.C + c];
        }
        cout_b[(size_t)r * p.C + c] = val;
      }
    }
  }

  const float scale_b = rbf(1.0f / sqrtf((float)kD));
  const float eps_b = rbf(1e-6f);

  for (int t0 = 0; t0 < T; t0 += kTC) {
    const int tc = min(kTC, T - t0);
    if (t0 > 0) __syncthreads();  // the previous pass is done reading LDS

    // ---- front end for steps t0 .. t0+tc-1 into LDS ----
    if (FE == 0) {
      float* q_s = reinterpret_cast<float*>(sm_q);
      float* k_s = reinterpret_cast<float*>(sm_k);
      const int per = 2 * kD + kTileRows;
      for (int e = tid; e < tc * per; e += kThreads) {
        const int tt = e / per;
        const int c = e % per;
        const size_t row = lb * T + (t0 + tt);
        if (c < kD) {
          q_s[tt * kD + c] = load_qkv(p.q, (row * p.Hk + g) * kD + c, p.qkv_bf16);
        } else if (c < 2 * kD) {
          k_s[tt * kD + c - kD] = load_qkv(p.k, (row * p.Hk + g) * kD + c - kD, p.qkv_bf16);
        } else {
          sm_v[tt][c - 2 * kD] = load_qkv(p.v, (row * p.Hv + h) * kD + r0 + c - 2 * kD, p.qkv_bf16);
        }
      }
    } else {
      if (wave < 2) {
        // wave 0: q of k-head g; wave 1: k. Lane l: channels l and l+64 of the head.
        float* dst = reinterpret_cast<float*>(wave == 0 ? sm_q : sm_k);
        const int cbase = (wave == 0 ? 0 : p.Hk * kD) + g * kD;
        for (int tt = 0; tt < tc; ++tt) {
          const int t = t0 + tt;
          const float u0 = silu_bf(conv_channel(x_b, cin_b, w_l, p.C, cbase + lane, t));
          const float u1 = silu_bf(conv_channel(x_b, cin_b, w_l, p.C, cbase + lane + 64, t));
          // l2norm (ops.cpp:27-30): x * rsqrt(sum(x*x) + eps), every op in bf16
          const float pr = rbf(u0 * u0) + rbf(u1 * u1);
          const float ssum = rbf(wave64_sum(pr));
          const float den = rbf(ssum + eps_b);
          const float rs = rbf(1.0f / sqrtf(den));
          float y0 = rbf(u0 * rs);
          float y1 = rbf(u1 * rs);
          if (wave == 0) {  // q *= 128^-0.5 (model.cpp:601)
            y0 = rbf(y0 * scale_b);
            y1 = rbf(y1 * scale_b);
          }
          dst[tt * kD + lane] = y0;
          dst[tt * kD + lane + 64] = y1;
        }
      } else if (wave == 2) {
        const int c = 2 * p.Hk * kD + h * kD + r0 + lane;
        for (int tt = 0; tt < tc; ++tt) {
          sm_v[tt][lane] = silu_bf(conv_channel(x_b, cin_b, w_l, p.C, c, t0 + tt));
        }
      }
    }
    // gates: one thread per step
    if (tid >= kThreads - kTC) {
      const int tt = tid - (kThreads - kTC);
      if (tt < tc) {
        const size_t gi = (lb * T + (t0 + tt)) * p.Hv + h;
        float al, be;
        if (p.gate_raw) {
          d_gates(bf2f(p.a[gi]), bf2f(p.b[gi]), p.A_log[(size_t)layer * p.Hv + h],
                  p.dt_bias[(size_t)layer * p.Hv + h], al, be);
        } else {
          al = p.alpha[gi];
          be = p.beta[gi];
        }
        sm_a[tt] = al;
        sm_b[tt] = be;
      }
    }
    __syncthreads();

    // ---- apply the steps to this wave's rows ----
    for (int tt = 0; tt < tc; ++tt) {
      const int t = t0 + tt;
      const float al = sm_a[tt];
      const float be = sm_b[tt];
      const float4 k0 = sm_k[tt][j16];
      const float4 k1 = sm_k[tt][16 + j16];
      const float4 q0 = sm_q[tt][j16];
      const float4 q1 = sm_q[tt][16 + j16];
      float ov[kSlots];
#pragma unroll
      for (int i = 0; i < kSlots; ++i) {
        const int rl = wave * 16 + i * 4 + grp;  // row within the tile
        const float vr = sm_v[tt][rl];
        float4& a0 = s[i][0];
        float4& a1 = s[i][1];
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
      if (COLLECT) {
        float* dst = p.states_tbh
                         ? p.states + ((((size_t)layer * T + t) * p.B + bb) * p.Hv + h) * DD
                         : p.states + (head * T + t) * DD;
#pragma unroll
        for (int i = 0; i < kSlots; ++i) {
          const int row = r0 + wave * 16 + i * 4 + grp;
          *reinterpret_cast<float4*>(dst + (size_t)row * kD + j16 * 4) = s[i][0];
          *reinterpret_cast<float4*>(dst + (size_t)row * kD + 64 + j16 * 4) = s[i][1];
        }
      }
      // lane j (< 4) of each group writes the output of slot j
      if (j16 < kSlots) {
        float val = ov[0];
        if (j16 == 1) val = ov[1];
        if (j16 == 2) val = ov[2];
        if (j16 == 3) val = ov[3];
        const int row = r0 + wave * 16 + j16 * 4 + grp;
        const size_t oi = ((lb * T + t) * p.Hv + h) * kD + row;
        if (p.o_bf16) {
          static_cast<uint16_t*>(p.o)[oi] = f2bf(val);
        } else {
          static_cast<float*>(p.o)[oi] = val;
        }
      }
    }
  }

  if (p.state_out) {
    float* sout = p.state_out + head * DD;
#pragma unroll
    for (int i = 0; i < kSlots; ++i) {
      const int row = r0 + wave * 16 + i * 4 + grp;
      *reinterpret_cast<float4*>(sout + (size_t)row * kD + j16 * 4) = s[i][0];
      *reinterpret_cast<float4*>(sout + (size_t)row * kD + 64 + j16 * 4) = s[i][1];
    }
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

}  // namespace

hipError_t launch_recurrent(const RecurrentParams& p, int frontend, bool collect,
                            hipStream_t stream) {
  const dim3 grid(p.nblocks), block(kThreads);
  if (frontend == 0) {
    if (collect) {
      hipLaunchKernelGGL((recurrent_kernel<0, true>), grid, block, 0, stream, p);
    } else {
      hipLaunchKernelGGL((recurrent_kernel<0, false>), grid, block, 0, stream, p);
    }
  } else {
    if (collect) {
      hipLaunchKernelGGL((recurrent_kernel<1, true>), grid, block, 0, stream, p);
    } else {
      hipLaunchKernelGGL((recurrent_kernel<1, false>), grid, block, 0, stream, p);
    }
  }
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

int recurrent_tile_rows() { return kTileRows; }

}  // namespace gdn
