// C++17 boundary test: drives include/infer/linear_hip.hpp and
// include/infer/linear_dispatch.hpp the way the reference's gtest suite
// drives include/infer/cuda_ops.hpp (tests/test_cuda.cpp), with a minimal
// in-file harness (no gtest in this image).  Expected values are float64
// closed forms computed here on the host.  Exit status 0 = all passed.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <vector>

#include "infer/linear_dispatch.hpp"

namespace {

int g_failures = 0;

#define EXPECT(cond, ...)                                   \
  do {                                                      \
    if (!(cond)) {                                          \
      ++g_failures;                                         \
      std::printf("FAIL %s:%d: ", __FILE__, __LINE__);      \
      std::printf(__VA_ARGS__);                             \
      std::printf("\n");                                    \
    }                                                       \
  } while (0)

uint16_t to_bf16(float v) {
  uint32_t b;
  std::memcpy(&b, &v, 4);
  b += 0x7FFFu + ((b >> 16) & 1u);
  return static_cast<uint16_t>(b >> 16);
}
float from_bf16(uint16_t w) {
  const uint32_t b = static_cast<uint32_t>(w) << 16;
  float v;
  std::memcpy(&v, &b, 4);
  return v;
}

template <typename T>
struct Dev {
  T* p{nullptr};
  size_t n{0};
  explicit Dev(const std::vector<T>& h) : n(h.size()) {
    infer::hip::check_hip(hipMalloc(&p, n * sizeof(T)), "hipMalloc");
    infer::hip::check_hip(hipMemcpy(p, h.data(), n * sizeof(T), hipMemcpyHostToDevice), "copy");
  }
  explicit Dev(size_t count) : n(count) {
    infer::hip::check_hip(hipMalloc(&p, n * sizeof(T)), "hipMalloc");
  }
  ~Dev() { (void)hipFree(p); }
  std::vector<T> host() const {
    std::vector<T> h(n);
    infer::hip::check_hip(hipMemcpy(h.data(), p, n * sizeof(T), hipMemcpyDeviceToHost), "copy");
    return h;
  }
};

// check_w8a16_linear_case generator, tests/test_cuda.cpp:519-557.
void w8a16_case(infer::hip::Context& ctx, int tokens, int n, int k, bool with_bias) {
  const int groups = (k + 63) / 64;
  std::vector<int8_t> q(static_cast<size_t>(n) * k);
  std::vector<uint16_t> s(static_cast<size_t>(n) * groups), x(static_cast<size_t>(tokens) * k),
      b(n);
  for (size_t i = 0; i < q.size(); ++i) q[i] = static_cast<int8_t>(static_cast<int>(i * 17 % 31) - 15);
  if (q.size() >= 2) { q[0] = -127; q[1] = 127; }
  for (size_t i = 0; i < s.size(); ++i) s[i] = to_bf16((1 + static_cast<int>(i % 7)) / 1024.0f);
  for (size_t i = 0; i < x.size(); ++i) x[i] = to_bf16((static_cast<int>(i * 13 % 29) - 14) / 64.0f);
  for (int r = 0; r < n; ++r) b[r] = to_bf16((r % 9 - 4) / 32.0f);
  if (k > 64) {
    std::fill_n(q.begin() + static_cast<size_t>(n - 1) * k, 64, static_cast<int8_t>(0));
    s[static_cast<size_t>(n - 1) * groups] = to_bf16(1.0f);
  }
  Dev<int8_t> dq(q);
  Dev<uint16_t> ds(s), dx(x), db(b), dy(static_cast<size_t>(tokens) * n), dv(n);
  const uint16_t* bias = with_bias ? db.p : nullptr;
  infer::hip::gemm_w8a16(dq.p, ds.p, 64, bias, dx.p, dy.p, tokens, n, k, ctx.stream());
  infer::hip::gemv_w8a16(dq.p, ds.p, 64, bias, dx.p, dv.p, n, k, ctx.stream());
  ctx.synchronize();
  const auto y = dy.host();
  const auto v = dv.host();
  for (int t = 0; t < tokens; ++t) {
    for (int r = 0; r < n; ++r) {
      double e = with_bias ? from_bf16(b[r]) : 0.0;
      for (int c = 0; c < k; ++c) {
        e += static_cast<double>(q[static_cast<size_t>(r) * k + c]) *
             from_bf16(s[static_cast<size_t>(r) * groups + c / 64]) *
             from_bf16(x[static_cast<size_t>(t) * k + c]);
      }
      const double got = from_bf16(y[static_cast<size_t>(t) * n + r]);
      const double tol = std::max(1.0 / 64, 0.01 * std::fabs(e));  // test_cuda.cpp:587-594
      EXPECT(std::fabs(got - e) <= tol, "w8a16 (%d,%d,%d) t=%d r=%d got %g want %g", tokens, n,
             k, t, r, got, e);
      if (t == 0) {
        EXPECT(std::fabs(from_bf16(v[r]) - got) <= std::max(1.0 / 64, 0.01 * std::fabs(got)),
               "gemv vs gemm row 0, r=%d", r);
      }
    }
  }
}

// check_bf16_linear_case generator, tests/test_cuda.cpp:621-642.
void bf16_case(infer::hip::Context& ctx, int tokens, int n, int k, bool with_bias) {
  std::vector<uint16_t> w(static_cast<size_t>(n) * k), x(static_cast<size_t>(tokens) * k), b(n);
  for (size_t i = 0; i < w.size(); ++i) w[i] = to_bf16((static_cast<int>(i % 17) - 8) * 0.015625f);
  for (size_t i = 0; i < x.size(); ++i) x[i] = to_bf16((static_cast<int>(i % 13) - 6) * 0.03125f);
  for (int r = 0; r < n; ++r) b[r] = to_bf16((r % 5 - 2) * 0.0625f);
  Dev<uint16_t> dw(w), dx(x), db(b), dy(static_cast<size_t>(tokens) * n);
  infer::hip::gemm_bf16(dw.p, with_bias ? db.p : nullptr, dx.p, dy.p, tokens, n, k, ctx.stream());
  ctx.synchronize();
  const auto y = dy.host();
  for (int t = 0; t < tokens; ++t) {
    for (int r = 0; r < n; ++r) {
      double e = with_bias ? from_bf16(b[r]) : 0.0;
      for (int c = 0; c < k; ++c) {
        e += static_cast<double>(from_bf16(w[static_cast<size_t>(r) * k + c])) *
             from_bf16(x[static_cast<size_t>(t) * k + c]);
      }
      const double got = from_bf16(y[static_cast<size_t>(t) * n + r]);
      EXPECT(std::fabs(got - e) <= std::max(0.004, 0.008 * std::fabs(e)),  // test_cuda.cpp:611-619
             "bf16 (%d,%d,%d) t=%d r=%d got %g want %g", tokens, n, k, t, r, got, e);
    }
  }
}

// check_lm_head_fused_case, tests/test_cuda.cpp:790-880.
void lm_head_case(infer::hip::Context& ctx, int vocab, int hidden, int tie_a, int tie_b) {
  std::vector<uint16_t> e(static_cast<size_t>(vocab) * hidden), h(hidden);
  for (size_t i = 0; i < e.size(); ++i) e[i] = to_bf16((static_cast<int>((i + 11) % 19) - 9) * 0.0078125f);
  for (int c = 0; c < hidden; ++c) {
    e[static_cast<size_t>(tie_a) * hidden + c] = to_bf16(2.0f);
    e[static_cast<size_t>(tie_b) * hidden + c] = to_bf16(2.0f);
    h[c] = to_bf16(c == 0 ? 100.0f : (c % 13 - 6) * 0.0234375f);
  }
  Dev<uint16_t> de(e), dh(h), dl(vocab);
  infer::LinearWeight embed{infer::DType::kBFloat16, de.p, nullptr, 0, nullptr, vocab, hidden};
  infer::hip::LmHeadWorkspace ws(vocab);
  EXPECT(infer::hip::lm_head_workspace_entries(vocab, hidden) <= static_cast<size_t>((vocab + 7) / 8),
         "workspace sizing");
  infer::hip::lm_head(embed, dh.p, dl.p, ws, ctx.stream());
  int argmax = -1;
  infer::hip::check_hip(hipMemcpyAsync(&argmax, ws.argmax(), sizeof(int), hipMemcpyDeviceToHost,
                                       ctx.stream()), "copy");
  ctx.synchronize();
  EXPECT(argmax == tie_a, "lm_head (%d,%d) argmax %d want %d", vocab, hidden, argmax, tie_a);
}

void dispatch_and_plan(infer::hip::Context& ctx) {
  // q/k/v-like weights on one input: the plan equals three dispatched calls.
  const int k = 896;
  const int ns[3] = {896, 128, 128};
  std::vector<Dev<int8_t>*> qs;
  std::vector<Dev<uint16_t>*> ss, ys, refs;
  std::vector<infer::LinearWeight> ws;
  std::vector<uint16_t> x(k);
  for (int c = 0; c < k; ++c) x[c] = to_bf16(std::sin(0.37f * c));
  Dev<uint16_t> dx(x);
  for (int i = 0; i < 3; ++i) {
    std::vector<int8_t> q(static_cast<size_t>(ns[i]) * k);
    std::vector<uint16_t> s(static_cast<size_t>(ns[i]) * (k / 64));
    for (size_t j = 0; j < q.size(); ++j) q[j] = static_cast<int8_t>((j * 7919 + i) % 255 - 127);
    for (size_t j = 0; j < s.size(); ++j) s[j] = to_bf16(1e-4f * (1 + j % 13));
    qs.push_back(new Dev<int8_t>(q));
    ss.push_back(new Dev<uint16_t>(s));
    ys.push_back(new Dev<uint16_t>(ns[i]));
    refs.push_back(new Dev<uint16_t>(ns[i]));
    ws.push_back({infer::DType::kInt8, qs.back()->p, ss.back()->p, 64, nullptr, ns[i], k});
    infer::hip::linear(ws.back(), dx.p, refs.back()->p, ctx.stream());
  }
  {
    auto plan = infer::hip::make_shared_input_plan({&ws[0], &ws[1], &ws[2]}, dx.p,
                                                   {ys[0]->p, ys[1]->p, ys[2]->p});
    plan.launch(ctx.stream());
    ctx.synchronize();
  }
  for (int i = 0; i < 3; ++i) {
    const auto a = ys[i]->host();
    const auto r = refs[i]->host();
    for (int j = 0; j < ns[i]; ++j) {
      const float fa = from_bf16(a[j]), fr = from_bf16(r[j]);
      EXPECT(std::fabs(fa - fr) <= 0.0079f * std::fabs(fr) + 1e-6f, "plan %d row %d: %g vs %g", i,
             j, fa, fr);
    }
    delete qs[i]; delete ss[i]; delete ys[i]; delete refs[i];
  }
  bool threw = false;
  try {
    infer::LinearWeight bad{infer::DType::kFloat32, dx.p, nullptr, 0, nullptr, 4, 4};
    infer::hip::linear(bad, dx.p, nullptr, ctx.stream());
  } catch (const infer::Error&) {
    threw = true;
  }
  EXPECT(threw, "FP32 weights must be rejected by the BF16 dispatch");
}

// linear_batch with a GemmWorkspace on a down_proj-shaped weight (K = 4864,
// split over K) equals the plain linear_batch within the reference's W8A16
// tolerance at several token counts sharing one workspace; a weight that
// never splits needs none.
void workspace_batch(infer::hip::Context& ctx) {
  const int n = 896, k = 4864, max_tokens = 64;
  std::vector<int8_t> q(static_cast<size_t>(n) * k);
  std::vector<uint16_t> s(static_cast<size_t>(n) * (k / 64)), x(static_cast<size_t>(max_tokens) * k);
  for (size_t j = 0; j < q.size(); ++j) q[j] = static_cast<int8_t>((j * 7919 + 3) % 255 - 127);
  for (size_t j = 0; j < s.size(); ++j) s[j] = to_bf16(1e-4f * (1 + j % 11));
  for (size_t j = 0; j < x.size(); ++j) x[j] = to_bf16(std::sin(0.013f * static_cast<float>(j)));
  Dev<int8_t> dq(q);
  Dev<uint16_t> ds(s), dx(x), dy(static_cast<size_t>(max_tokens) * n),
      dr(static_cast<size_t>(max_tokens) * n);
  const infer::LinearWeight w{infer::DType::kInt8, dq.p, ds.p, 64, nullptr, n, k};
  const infer::LinearWeight shortk{infer::DType::kInt8, dq.p, ds.p, 64, nullptr, n, 896};
  infer::hip::GemmWorkspace ws(max_tokens, {&w});
  infer::hip::GemmWorkspace none(max_tokens, {&shortk});
  EXPECT(ws.bytes() > 0, "a K = 4864 weight splits at %d tokens", max_tokens);
  EXPECT(none.bytes() == 0, "a K = 896 weight needs no workspace (%zu bytes)", none.bytes());
  for (int tokens : {2, 33, 64, 17}) {
    infer::hip::linear_batch(w, dx.p, dy.p, tokens, ws, ctx.stream());
    infer::hip::linear_batch(w, dx.p, dr.p, tokens, ctx.stream());
    ctx.synchronize();
    const auto a = dy.host(), r = dr.host();
    int bad = 0;
    for (size_t j = 0; j < static_cast<size_t>(tokens) * n; ++j) {
      const float fa = from_bf16(a[j]), fr = from_bf16(r[j]);
      bad += !(std::fabs(fa - fr) <= std::max(1.0f / 64, 0.01f * std::fabs(fr)));
    }
    EXPECT(bad == 0, "workspace linear_batch at %d tokens: %d outputs off", tokens, bad);
  }
  bool threw = false;
  try {  // a workspace smaller than the call needs
    infer::hip::gemm_w8a16(dq.p, ds.p, 64, nullptr, dx.p, dy.p, max_tokens, n, k, ws.data(), 16,
                           ctx.stream());
  } catch (const infer::Error& e) {
    threw = std::strstr(e.what(), "workspace") != nullptr;
  }
  EXPECT(threw, "a too small workspace must throw infer::Error");
}

}  // namespace

int main() {
  try {
    infer::hip::Context ctx;
    bool threw = false;
    try {  // tests/test_cuda.cpp:887-890
      infer::hip::gemv_w8a16(nullptr, nullptr, 32, nullptr, nullptr, nullptr, 1, 1, ctx.stream());
    } catch (const infer::Error& e) {
      threw = std::strstr(e.what(), "group size must be 64") != nullptr;
    }
    EXPECT(threw, "group size 32 must throw infer::Error");
    w8a16_case(ctx, 3, 5, 70, true);
    w8a16_case(ctx, 2, 7, 65, false);
    w8a16_case(ctx, 2, 896, 896, true);
    w8a16_case(ctx, 2, 896, 4864, false);
    bf16_case(ctx, 3, 11, 14, true);
    bf16_case(ctx, 32, 64, 64, true);
    bf16_case(ctx, 65, 70, 67, false);
    lm_head_case(ctx, 512, 64, 3, 4);
    lm_head_case(ctx, 1002, 64, 7, 71);
    lm_head_case(ctx, 64, 896, 1, 31);
    dispatch_and_plan(ctx);
    workspace_batch(ctx);
  } catch (const std::exception& e) {
    std::printf("FAIL: exception %s\n", e.what());
    return 2;
  }
  std::printf("%s: %d failure(s)\n", g_failures ? "FAILED" : "PASSED", g_failures);
  return g_failures ? 1 : 0;
}
