// C++ host-side test of libgdn.so through include/gdn.hpp, in the style of the
// reference's self-test (cpp/src/tests.cpp:36-56 rel_err/check, 196-243 test_delta):
// gdn::run vs the oracle's run_reference restatement on the reference's shapes and input
// distributions, with and without collect, bound 2e-5; then DeltaCache record/commit
// against plain decoding; then the quantized projections (gdn::linears, norm_out_proj). The oracle (oracle/gdn_oracle.h) is used for comparison only.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "gdn.hpp"
#include "gdn_oracle.h"

namespace {

int g_pass = 0, g_fail = 0;

void check(bool ok, const std::string& what) {
  printf("  [%s] %s\n", ok ? "ok" : "FAIL", what.c_str());
  (ok ? g_pass : g_fail)++;
}

// max|a-b| / max|b| (tests.cpp:38-45)
float rel_err(const std::vector<float>& a, const std::vector<float>& b) {
  float num = 0.f, den = 0.f;
  for (size_t i = 0; i < a.size(); ++i) {
    num = std::max(num, std::fabs(a[i] - b[i]));
    den = std::max(den, std::fabs(b[i]));
  }
  return num / (den > 0 ? den : 1.0f);
}

template <class T>
T* to_dev(const std::vector<T>& h) {
  T* d = nullptr;
  gdn::check_hip(hipMalloc(&d, h.size() * sizeof(T)), "hipMalloc");
  gdn::check_hip(hipMemcpy(d, h.data(), h.size() * sizeof(T), hipMemcpyHostToDevice), "copy");
  return d;
}

template <class T>
std::vector<T> to_host(const T* d, size_t n) {
  std::vector<T> h(n);
  gdn::check_hip(hipMemcpy(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost), "copy");
  return h;
}

std::vector<float> normal(uint64_t seed, size_t n, float std = 1.0f) {
  std::vector<float> v(n);
  gdno_fill_normal(seed, 0.0f, std, v.data(), (int64_t)n);
  return v;
}

void l2norm_rows(std::vector<float>& x, float scale) {
  for (size_t r = 0; r < x.size() / 128; ++r) {
    double s = 0;
    for (int d = 0; d < 128; ++d) s += (double)x[r * 128 + d] * x[r * 128 + d];
    const double inv = scale / std::sqrt(s);
    for (int d = 0; d < 128; ++d) x[r * 128 + d] = (float)(x[r * 128 + d] * inv);
  }
}

void test_delta() {
  printf("\ndelta kernel (gfx950 available: %s)\n", gdn::available() ? "yes" : "no");
  struct Case {
    int B, L, H;
  };
  for (const Case& c : {Case{1, 1, 48}, Case{1, 4, 48}, Case{1, 9, 48}, Case{2, 3, 16},
                        Case{1, 64, 48}, Case{1, 384, 8}}) {
    const size_t nq = (size_t)c.B * c.L * c.H * 128, ng = (size_t)c.B * c.L * c.H,
                 ns = (size_t)c.B * c.H * 128 * 128;
    const uint64_t s = 9000 + 7 * c.L + c.H;
    auto q = normal(s, nq), k = normal(s + 1, nq), v = normal(s + 2, nq), S0 = normal(s + 5, ns, 0.1f);
    l2norm_rows(q, 1.0f / std::sqrt(128.0f));
    l2norm_rows(k, 1.0f);
    std::vector<float> al(ng), bt(ng);
    gdno_fill_uniform(s + 3, 0.85f, 1.0f, al.data(), (int64_t)ng);
    gdno_fill_uniform(s + 4, 0.0f, 1.0f, bt.data(), (int64_t)ng);

    std::vector<float> ro(nq), rS(ns), rst(ns * c.L);
    gdno_recurrent_f32(c.B, c.L, c.H, c.H, q.data(), k.data(), v.data(), al.data(), bt.data(),
                       S0.data(), rS.data(), ro.data(), rst.data(), 0, 0);

    float *dq = to_dev(q), *dk = to_dev(k), *dv = to_dev(v), *da = to_dev(al), *db = to_dev(bt),
          *dS = to_dev(S0), *dO, *dSo, *dSt;
    gdn::check_hip(hipMalloc(&dO, nq * 4), "hipMalloc");
    gdn::check_hip(hipMalloc(&dSo, ns * 4), "hipMalloc");
    gdn::check_hip(hipMalloc(&dSt, ns * c.L * 4), "hipMalloc");
    gdn::run(c.B, c.L, c.H, dq, dk, dv, da, db, dS, dO, dSo);
    gdn::check_hip(hipDeviceSynchronize(), "sync");
    const float eo = rel_err(to_host(dO, nq), ro), es = rel_err(to_host(dSo, ns), rS);
    char buf[160];
    snprintf(buf, sizeof(buf), "B=%d L=%3d H=%2d  out %.2e  state %.2e", c.B, c.L, c.H, eo, es);
    check(std::max(eo, es) < 2e-5f, buf);

    gdn::run(c.B, c.L, c.H, dq, dk, dv, da, db, dS, dO, nullptr, dSt);
    gdn::check_hip(hipDeviceSynchronize(), "sync");
    const float ec = rel_err(to_host(dSt, ns * c.L), rst);
    snprintf(buf, sizeof(buf), "  collect: %d states, max rel err %.2e", c.L, ec);
    check(ec < 2e-5f, buf);
    for (float* p : {dq, dk, dv, da, db, dS, dO, dSo, dSt}) (void)hipFree(p);
  }
}

// DeltaCache record/commit against plain decoding of the accepted prefix
// (session.cpp:476-515 contract), and step() against the oracle's layer sequence.
void test_cache() {
  printf("\nDeltaCache (record / commit)\n");
  const int B = 2, Hk = 16, Hv = 48, C = 2 * Hk * 128 + Hv * 128, T = 5;
  std::vector<uint16_t> w(4 * C), x((size_t)B * (T + 1) * C), a((size_t)B * (T + 1) * Hv),
      b((size_t)B * (T + 1) * Hv);
  gdno_round_bf16(normal(11, w.size(), 0.1f).data(), w.data(), (int64_t)w.size());
  gdno_round_bf16(normal(12, x.size()).data(), x.data(), (int64_t)x.size());
  gdno_round_bf16(normal(13, a.size()).data(), a.data(), (int64_t)a.size());
  gdno_round_bf16(normal(14, b.size()).data(), b.data(), (int64_t)b.size());
  std::vector<float> A_log(Hv), dt = normal(16, Hv, 0.1f);
  gdno_fill_uniform(15, -1.0f, 1.0f, A_log.data(), Hv);
  uint16_t *dw = to_dev(w), *dx = to_dev(x), *da = to_dev(a), *db = to_dev(b);
  float *dA = to_dev(A_log), *ddt = to_dev(dt);
  gdn::LayerParams p;
  p.conv_weight = dw;
  p.A_log = dA;
  p.dt_bias = ddt;
  uint16_t* o;
  gdn::check_hip(hipMalloc(&o, (size_t)B * T * Hv * 128 * 2), "hipMalloc");

  // per-token slices of x, a, b: (B, 1, .) rows of a (B, T+1, .) buffer are not
  // contiguous for B > 1, so copy each token to its own buffer
  auto token = [&](const std::vector<uint16_t>& src, int t, int width) {
    std::vector<uint16_t> h((size_t)B * width);
    for (int bb = 0; bb < B; ++bb)
      memcpy(&h[(size_t)bb * width], &src[((size_t)bb * (T + 1) + t) * width], width * 2);
    return to_dev(h);
  };
  auto block = [&](const std::vector<uint16_t>& src, int t0, int n, int width) {
    std::vector<uint16_t> h((size_t)B * n * width);
    for (int bb = 0; bb < B; ++bb)
      memcpy(&h[(size_t)bb * n * width], &src[((size_t)bb * (T + 1) + t0) * width], (size_t)n * width * 2);
    return to_dev(h);
  };
  // two speculative rounds in a row (the block is tokens 0..T-1 both times): the first
  // commit adopts its state by pointer, the second block is recorded into the other buffer
  const int rounds[4][2] = {{0, 3}, {2, 5}, {5, 1}, {3, 0}};
  for (const auto& jj : rounds) {
    gdn::DeltaCache spec(p, B, T), plain(p, B, 0);
    uint16_t* xb = block(x, 0, T, C);
    uint16_t* ab = block(a, 0, T, Hv);
    uint16_t* bb_ = block(b, 0, T, Hv);
    bool swapped = true;
    for (int j : jj) {
      const float* before = spec.state();
      spec.record = true;
      spec.step(xb, ab, bb_, T, o, nullptr);
      spec.commit(j, nullptr);
      swapped = swapped && ((j > 0) == (spec.state() != before));
      for (int t = 0; t < j; ++t) {
        uint16_t *xt = token(x, t, C), *at = token(a, t, Hv), *bt = token(b, t, Hv);
        plain.step(xt, at, bt, 1, o, nullptr);
        gdn::check_hip(hipDeviceSynchronize(), "sync");
        (void)hipFree(xt); (void)hipFree(at); (void)hipFree(bt);
      }
    }
    uint16_t *xt = token(x, T, C), *at = token(a, T, Hv), *bt = token(b, T, Hv);
    spec.step(xt, at, bt, 1, o, nullptr);
    plain.step(xt, at, bt, 1, o, nullptr);
    gdn::check_hip(hipDeviceSynchronize(), "sync");
    const auto s1 = to_host(spec.state(), spec.state_bytes() / 4);
    const auto s2 = to_host(plain.state(), plain.state_bytes() / 4);
    const auto c1 = to_host((const uint16_t*)spec.conv(), spec.conv_bytes() / 2);
    const auto c2 = to_host((const uint16_t*)plain.conv(), plain.conv_bytes() / 2);
    char buf[200];
    snprintf(buf, sizeof(buf),
             "commit(%d), commit(%d) then one step == plain decoding of %d + %d tokens (offset %d)", jj[0],
             jj[1], jj[0], jj[1], spec.offset);
    check(s1 == s2 && c1 == c2 && spec.offset == plain.offset && spec.offset == jj[0] + jj[1] + 1, buf);
    check(swapped, "commit(n > 0) adopts the recorded state by pointer, commit(0) keeps the state");
    for (uint16_t* ptr : {xb, ab, bb_, xt, at, bt}) (void)hipFree(ptr);
  }
  bool threw = false;
  try {
    gdn::DeltaCache c(p, B, T);
    uint16_t* xb = block(x, 0, T, C);
    uint16_t* ab = block(a, 0, T, Hv);
    uint16_t* bb_ = block(b, 0, T, Hv);
    c.record = true;
    c.step(xb, ab, bb_, T, o, nullptr);
    c.commit(T + 1, nullptr);
  } catch (const gdn::Error&) {
    threw = true;
  }
  check(threw, "commit out of range throws (model.cpp:443)");
}

// A block of chunked_min_t(B) .. max_prefill_tokens tokens runs the chunked form
// (python/qwen35.py:606-626 chooses by length the same way): against a cache without a
// prefill workspace, which runs the same block on the recurrent kernel, within the chunked
// form's tolerance (1e-2); the conv window is exact in both forms.
void test_cache_chunked() {
  printf("\nDeltaCache: long block on the chunked form\n");
  const int B = 2, Hk = 16, Hv = 48, C = 2 * Hk * 128 + Hv * 128, T = 40;
  std::vector<uint16_t> w(4 * C), x((size_t)B * T * C), a((size_t)B * T * Hv), b((size_t)B * T * Hv);
  gdno_round_bf16(normal(21, w.size(), 0.1f).data(), w.data(), (int64_t)w.size());
  gdno_round_bf16(normal(22, x.size()).data(), x.data(), (int64_t)x.size());
  gdno_round_bf16(normal(23, a.size()).data(), a.data(), (int64_t)a.size());
  gdno_round_bf16(normal(24, b.size()).data(), b.data(), (int64_t)b.size());
  std::vector<float> A_log(Hv), dt = normal(26, Hv, 0.1f);
  gdno_fill_uniform(25, -1.0f, 1.0f, A_log.data(), Hv);
  uint16_t *dw = to_dev(w), *dx = to_dev(x), *da = to_dev(a), *db = to_dev(b);
  float *dA = to_dev(A_log), *ddt = to_dev(dt);
  gdn::LayerParams p;
  p.conv_weight = dw;
  p.A_log = dA;
  p.dt_bias = ddt;
  uint16_t *o1, *o2;
  gdn::check_hip(hipMalloc(&o1, (size_t)B * T * Hv * 128 * 2), "hipMalloc");
  gdn::check_hip(hipMalloc(&o2, (size_t)B * T * Hv * 128 * 2), "hipMalloc");
  gdn::DeltaCache chunked(p, B, 0, 1024), recurrent(p, B, 0);
  chunked.step(dx, da, db, T, o1, nullptr);
  recurrent.step(dx, da, db, T, o2, nullptr);
  gdn::check_hip(hipDeviceSynchronize(), "sync");
  const auto s1 = to_host(chunked.state(), chunked.state_bytes() / 4);
  const auto s2 = to_host(recurrent.state(), recurrent.state_bytes() / 4);
  const auto c1 = to_host((const uint16_t*)chunked.conv(), chunked.conv_bytes() / 2);
  const auto c2 = to_host((const uint16_t*)recurrent.conv(), recurrent.conv_bytes() / 2);
  const auto h1 = to_host(o1, (size_t)B * T * Hv * 128), h2 = to_host(o2, (size_t)B * T * Hv * 128);
  std::vector<float> f1(h1.size()), f2(h2.size());
  for (size_t i = 0; i < h1.size(); ++i) {
    uint32_t u1 = (uint32_t)h1[i] << 16, u2 = (uint32_t)h2[i] << 16;
    memcpy(&f1[i], &u1, 4);
    memcpy(&f2[i], &u2, 4);
  }
  const float es = rel_err(s1, s2), eo = rel_err(f1, f2);
  char buf[200];
  snprintf(buf, sizeof(buf), "T=%d block: chunked vs recurrent state %.2e, o %.2e (<= 1e-2), conv window exact",
           T, es, eo);
  check(es <= 1e-2f && eo <= 1e-2f && c1 == c2 && chunked.offset == T, buf);
  for (void* ptr : {(void*)dw, (void*)dx, (void*)da, (void*)db, (void*)dA, (void*)ddt, (void*)o1, (void*)o2})
    (void)hipFree(ptr);
}

}  // namespace

// gdn::linears (the layer's four in_proj matrices on one x) and gdn::norm_out_proj vs the
// oracle's fp64 dequantize-and-dot: within half a bf16 ulp plus the fp32 accumulation.
void test_qlinear() {
  printf("quantized linear (model.cpp:356-372)\n");
  const int M = 1, K = 5120;
  const int ns[4] = {256, 96, 48, 48};
  uint64_t st = 12345;
  std::vector<uint16_t> x(M * K);
  {
    std::vector<float> xf = normal(501, x.size());
    gdno_round_bf16(xf.data(), x.data(), (int64_t)x.size());
  }
  uint16_t* dx = to_dev(x);
  std::vector<gdn::QuantLinear> W(4);
  std::vector<void*> y(4);
  std::vector<std::vector<uint32_t>> hw(4);
  std::vector<std::vector<uint16_t>> hs(4), hb(4);
  for (int i = 0; i < 4; ++i) {
    const int N = ns[i];
    hw[i].resize((size_t)N * K / 8);
    for (auto& v : hw[i]) v = (uint32_t)gdno_splitmix64_next(&st);
    std::vector<float> sf(N * K / 64), bf(N * K / 64);
    gdno_fill_uniform(600 + i, 0.002f, 0.03f, sf.data(), (int64_t)sf.size());
    gdno_fill_uniform(700 + i, -0.2f, 0.2f, bf.data(), (int64_t)bf.size());
    hs[i].resize(sf.size());
    hb[i].resize(bf.size());
    gdno_round_bf16(sf.data(), hs[i].data(), (int64_t)sf.size());
    gdno_round_bf16(bf.data(), hb[i].data(), (int64_t)bf.size());
    W[i] = gdn::QuantLinear{to_dev(hw[i]), to_dev(hs[i]), to_dev(hb[i]), N};
    gdn::check_hip(hipMalloc(&y[i], (size_t)M * N * 2), "hipMalloc");
  }
  gdn::linears(M, K, dx, W.data(), y.data(), 4);
  gdn::check_hip(hipDeviceSynchronize(), "sync");
  for (int i = 0; i < 4; ++i) {
    const int N = ns[i];
    std::vector<double> ref((size_t)M * N);
    gdno_qlinear_f64(M, N, K, x.data(), hw[i].data(), hs[i].data(), hb[i].data(), ref.data());
    std::vector<uint16_t> got = to_host(static_cast<uint16_t*>(y[i]), (size_t)M * N);
    double worst = 0;
    for (int n = 0; n < N; ++n) {
      double acc = 0;  // 2^-20 sum |x| (143 |s| + |b|)
      for (int k = 0; k < K; ++k)
        acc += std::fabs(gdno_bf16_to_f32(x[k])) * (143.0 * std::fabs(gdno_bf16_to_f32(hs[i][(size_t)n * K / 64 + k / 64])) +
                                                   std::fabs(gdno_bf16_to_f32(hb[i][(size_t)n * K / 64 + k / 64])));
      const double lim = std::ldexp(std::fabs(ref[n]), -8) + std::ldexp(acc, -20);
      worst = std::max(worst, std::fabs(gdno_bf16_to_f32(got[n]) - ref[n]) / lim);
    }
    char buf[128];
    snprintf(buf, sizeof(buf), "in_proj segment %d (N=%d): worst err / limit %.3f", i, N, worst);
    check(worst <= 1.0, buf);
  }
  // norm + out_proj
  {
    const int Ko = 6144, No = 64;
    std::vector<float> o = normal(801, (size_t)M * Ko, 0.3f), zf = normal(802, (size_t)M * Ko);
    std::vector<uint16_t> z(zf.size());
    gdno_round_bf16(zf.data(), z.data(), (int64_t)z.size());
    std::vector<float> gamma(128);
    gdno_fill_uniform(803, 0.5f, 1.5f, gamma.data(), 128);
    std::vector<uint32_t> w((size_t)No * Ko / 8);
    for (auto& v : w) v = (uint32_t)gdno_splitmix64_next(&st);
    std::vector<float> sf(No * Ko / 64, 0.01f), bf(No * Ko / 64, 0.05f);
    std::vector<uint16_t> sh(sf.size()), bh(bf.size());
    gdno_round_bf16(sf.data(), sh.data(), (int64_t)sf.size());
    gdno_round_bf16(bf.data(), bh.data(), (int64_t)bf.size());
    gdn::QuantLinear Wo{to_dev(w), to_dev(sh), to_dev(bh), No};
    float* dout = nullptr;
    gdn::check_hip(hipMalloc(&dout, (size_t)M * No * 2), "hipMalloc");
    gdn::norm_out_proj(Wo, M, Ko, to_dev(o), to_dev(z), to_dev(gamma), 1e-6f, dout);
    gdn::check_hip(hipDeviceSynchronize(), "sync");
    std::vector<uint16_t> xn((size_t)M * Ko);
    gdno_gated_rmsnorm((int64_t)M * Ko / 128, 128, o.data(), z.data(), gamma.data(), 1e-6f, xn.data());
    std::vector<double> ref((size_t)M * No);
    gdno_qlinear_f64(M, No, Ko, xn.data(), w.data(), sh.data(), bh.data(), ref.data());
    std::vector<uint16_t> got = to_host(reinterpret_cast<uint16_t*>(dout), (size_t)M * No);
    double xmax = 0;
    for (uint16_t v : xn) xmax = std::max(xmax, (double)std::fabs(gdno_bf16_to_f32(v)));
    double worst = 0;
    for (int n = 0; n < No; ++n) {
      // bf16 rounding, accumulation, and up to 3 one-ulp operand flips between the norms
      const double lim = std::ldexp(std::fabs(ref[n]), -8) + 1e-3 * xmax + 3 * std::ldexp(xmax * (15 * 0.01 + 0.05), -8);
      worst = std::max(worst, std::fabs(gdno_bf16_to_f32(got[n]) - ref[n]) / lim);
    }
    char buf[128];
    snprintf(buf, sizeof(buf), "GatedRMSNorm + out_proj (N=%d, K=%d): worst err / limit %.3f", No, Ko, worst);
    check(worst <= 1.0, buf);
  }
  // a verify block's rows (M = 40): the MFMA path, with a caller workspace
  {
    const int Mv = 40, N = ns[0];
    std::vector<float> xf = normal(901, (size_t)Mv * K);
    std::vector<uint16_t> xv(xf.size());
    gdno_round_bf16(xf.data(), xv.data(), (int64_t)xv.size());
    const size_t ws_bytes = gdn::qlinear_workspace_size(Mv, K);
    void* ws = nullptr;
    gdn::check_hip(hipMalloc(&ws, ws_bytes), "hipMalloc");
    void* yv = nullptr;
    gdn::check_hip(hipMalloc(&yv, (size_t)Mv * N * 2), "hipMalloc");
    gdn::linear(W[0], Mv, K, to_dev(xv), yv, nullptr, ws, ws_bytes);
    gdn::check_hip(hipDeviceSynchronize(), "sync");
    std::vector<double> ref((size_t)Mv * N);
    gdno_qlinear_f64(Mv, N, K, xv.data(), hw[0].data(), hs[0].data(), hb[0].data(), ref.data());
    std::vector<uint16_t> got = to_host(static_cast<uint16_t*>(yv), (size_t)Mv * N);
    double worst = 0;
    for (int m = 0; m < Mv; ++m)
      for (int n = 0; n < N; ++n) {
        double acc = 0;  // 2^-20 sum |x| (143 |s| + |b|)
        for (int k = 0; k < K; ++k)
          acc += std::fabs(gdno_bf16_to_f32(xv[(size_t)m * K + k])) *
                 (143.0 * std::fabs(gdno_bf16_to_f32(hs[0][(size_t)n * K / 64 + k / 64])) +
                  std::fabs(gdno_bf16_to_f32(hb[0][(size_t)n * K / 64 + k / 64])));
        const double r = ref[(size_t)m * N + n];
        const double lim = std::ldexp(std::fabs(r), -8) + std::ldexp(acc, -20);
        worst = std::max(worst, std::fabs(gdno_bf16_to_f32(got[(size_t)m * N + n]) - r) / lim);
      }
    char buf[128];
    snprintf(buf, sizeof(buf), "M=%d rows (MFMA path, workspace %zu B): worst err / limit %.3f", Mv, ws_bytes, worst);
    check(worst <= 1.0, buf);
    bool threw = false;
    try {
      gdn::linear(W[0], Mv, K, to_dev(xv), yv);  // no workspace
    } catch (const gdn::Error&) {
      threw = true;
    }
    check(threw, "M=40 without a workspace throws");
  }
}

int main() {
  if (!gdn::available()) {
    printf("[skip] no gfx950 device\n");
    return 0;
  }
  try {
    test_delta();
    test_cache();
    test_cache_chunked();
    test_qlinear();
  } catch (const std::exception& e) {
    printf("  [FAIL] exception: %s\n", e.what());
    ++g_fail;
  }
  printf("\n%d passed, %d failed\n", g_pass, g_fail);
  return g_fail == 0 ? 0 : 1;
}
