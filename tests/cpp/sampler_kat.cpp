// sampler_kat.cpp -- known-answer tests of the C++ sampler wrapper
// (mlxforge_amd/include/mlxforge_amd/sampler.hpp) on the GPU.
//
// The cases are those of the reference's tests/sample/sampler_test.cpp, held
// on the same tiny logits and the same expected answers, but run through
// mlxforge_amd::Sampler on device buffers.  Two changes follow from the
// boundary:
//   * the MLX PRNG key becomes one caller-supplied uniform per row, so
//     "same seed reproduces" is "same uniforms reproduce";
//   * the kept sets of top-k / top-p / min_p are checked twice: through the
//     draw (a uniform sweep only ever returns kept ids, and reaches every one
//     of them) and directly, through the filter entry points apply_top_k /
//     apply_top_p / apply_min_p, on the reference's own cases.
// The reference's min_p and penalty cases (sampler_test.cpp:76-124) run through
// the wrapper's min_p parameter and apply_penalties; penalties left in the
// parameters of a sampling call must be refused.  The C ABI's seeded uniforms
// and grammar mask are checked on their own known answers.
//
// Prints one line per case and exits non-zero on the first failure set.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <set>
#include <string>
#include <vector>

#include "mlxforge_amd/sampler.hpp"

using mlxforge_amd::DeviceLogits;
using mlxforge_amd::Sampler;
using mlxforge_amd::SamplerError;
using mlxforge_amd::SamplingParams;
using mlxforge_amd::SampleResult;

namespace {

int g_failures = 0;
int g_checks = 0;

#define KAT_CHECK(cond)                                                            \
  do {                                                                             \
    ++g_checks;                                                                    \
    if (!(cond)) {                                                                 \
      ++g_failures;                                                                \
      std::fprintf(stderr, "  FAILED %s:%d: %s\n", __FILE__, __LINE__, #cond);     \
    }                                                                              \
  } while (0)

// A [B, V] fp32 matrix uploaded to the device for the lifetime of the object.
struct Logits {
  float* d = nullptr;
  int B = 0, V = 0;
  explicit Logits(const std::vector<std::vector<float>>& rows) {
    B = static_cast<int>(rows.size());
    V = static_cast<int>(rows[0].size());
    std::vector<float> flat;
    for (const auto& r : rows) flat.insert(flat.end(), r.begin(), r.end());
    if (hipMalloc(reinterpret_cast<void**>(&d), flat.size() * sizeof(float)) != hipSuccess ||
        hipMemcpy(d, flat.data(), flat.size() * sizeof(float), hipMemcpyHostToDevice) != hipSuccess) {
      std::fprintf(stderr, "device upload failed\n");
      std::exit(2);
    }
  }
  ~Logits() { (void)hipFree(d); }
  DeviceLogits view() const { return DeviceLogits{d, MLXF_DTYPE_F32, B, V, 0}; }
};

std::vector<float> log_of(const std::vector<float>& probs) {
  std::vector<float> lg(probs.size());
  for (size_t i = 0; i < probs.size(); ++i) lg[i] = std::log(probs[i]);
  return lg;
}

// Ids a single-row sample returns over a sweep of uniforms in [0, 1).
std::set<int> kept_by_sweep(Sampler& s, const Logits& lg, const SamplingParams& p, int n) {
  std::set<int> seen;
  std::vector<SamplingParams> rows(1, p);
  for (int i = 0; i < n; ++i) {
    const float u = (static_cast<float>(i) + 0.5f) / static_cast<float>(n);
    SampleResult r = s.sample_rows(lg.view(), rows, {u});
    seen.insert(r.tokens[0]);
  }
  return seen;
}

void case_greedy(Sampler& s) {  // sampler_test.cpp:41-44
  Logits lg({{1.0f, 3.0f, 2.0f}, {5.0f, 0.0f, -1.0f}});
  std::vector<int32_t> ids = s.greedy(lg.view());
  KAT_CHECK((ids == std::vector<int32_t>{1, 0}));
}

void case_temperature_zero(Sampler& s) {  // :46-52
  Logits lg({{0.2f, 0.9f, 0.1f, 0.4f}});
  SamplingParams p;
  p.temperature = 0.0f;
  SampleResult r = s.sample(lg.view(), p, {0.37f});
  KAT_CHECK(r.tokens == s.greedy(lg.view()));
}

void case_top_k(Sampler& s) {  // :54-61
  Logits lg({{5.0f, 1.0f, 4.0f, 2.0f, 3.0f}});
  SamplingParams p;
  p.top_k = 2;
  std::set<int> kept = kept_by_sweep(s, lg, p, 64);
  KAT_CHECK((kept == std::set<int>{0, 2}));
  // The draw splits at w(4) / (w(5) + w(4)) in ascending vocabulary order:
  // u below 1 / (1 + e^-1) picks id 0, above it id 2.
  std::vector<SamplingParams> rows(1, p);
  KAT_CHECK(s.sample_rows(lg.view(), rows, {0.70f}).tokens[0] == 0);
  KAT_CHECK(s.sample_rows(lg.view(), rows, {0.76f}).tokens[0] == 2);
}

void case_top_p(Sampler& s) {  // :63-74
  Logits lg({log_of({0.5f, 0.3f, 0.15f, 0.05f})});
  SamplingParams p;
  p.top_p = 0.7f;
  std::set<int> kept = kept_by_sweep(s, lg, p, 64);
  KAT_CHECK((kept == std::set<int>{0, 1}));
}

void case_reproducible(Sampler& s) {  // :126-134, with uniforms in place of keys
  std::vector<std::vector<float>> zeros(64, std::vector<float>(16, 0.0f));
  Logits lg(zeros);
  SamplingParams p;  // temperature 1, no top-k / top-p
  std::mt19937 g42(42), g7(7);
  std::uniform_real_distribution<float> U(0.0f, 1.0f);
  std::vector<float> u42(64), u7(64);
  for (auto& x : u42) x = U(g42);
  for (auto& x : u7) x = U(g7);
  std::vector<int32_t> a1 = s.sample(lg.view(), p, u42).tokens;
  std::vector<int32_t> a2 = s.sample(lg.view(), p, u42).tokens;
  std::vector<int32_t> b = s.sample(lg.view(), p, u7).tokens;
  KAT_CHECK(a1 == a2);
  KAT_CHECK(a1 != b);
  // Uniform logits: the inverse CDF is floor(u * 16).
  bool exact = true;
  for (int r = 0; r < 64; ++r) exact &= a1[r] == static_cast<int>(std::floor(u42[r] * 16.0f));
  KAT_CHECK(exact);
}

void case_batched(Sampler& s) {  // :136-142
  Logits lg({{1.0f, 2.0f, 3.0f}, {3.0f, 2.0f, 1.0f}});
  SampleResult r = s.sample(lg.view(), SamplingParams{}, {0.2f, 0.9f});
  KAT_CHECK(r.tokens.size() == 2 && r.logprobs.size() == 2);
  for (float lp : r.logprobs) KAT_CHECK(lp <= 0.0f);
}

void case_top_logprobs_off(Sampler& s) {  // :144-150
  Logits lg({{1.0f, 2.0f, 3.0f}});
  std::vector<SamplingParams> rows(1);  // top_logprobs = -1
  SampleResult r = s.sample_rows(lg.view(), rows, {0.5f});
  KAT_CHECK(r.K == 0 && r.top_tokens.empty() && r.top_logprobs.empty());
}

void case_top_logprobs_zero(Sampler& s) {  // :152-161
  Logits lg({{1.0f, 2.0f, 3.0f}});
  SamplingParams p;
  p.temperature = 0.0f;
  p.top_logprobs = 0;
  SampleResult r = s.sample(lg.view(), p, {0.5f});
  KAT_CHECK((r.tokens == std::vector<int32_t>{2}));
  KAT_CHECK(r.logprobs[0] <= 0.0f);
  KAT_CHECK(r.K == 0 && r.top_tokens.empty());
}

void case_top_logprobs_ranked(Sampler& s) {  // :163-181
  Logits lg({{1.0f, 4.0f, 2.0f, 3.0f, 0.0f}});
  SamplingParams p;
  p.temperature = 0.0f;
  p.top_logprobs = 3;
  SampleResult r = s.sample(lg.view(), p, {0.5f});
  KAT_CHECK(r.K == 3);
  KAT_CHECK((r.top_tokens == std::vector<int32_t>{1, 3, 2}));
  KAT_CHECK(r.top_logprobs[0] >= r.top_logprobs[1] && r.top_logprobs[1] >= r.top_logprobs[2]);
  for (float x : r.top_logprobs) KAT_CHECK(x <= 0.0f);
  KAT_CHECK((r.tokens == std::vector<int32_t>{1}));
  KAT_CHECK(std::fabs(r.logprobs[0] - r.top_logprobs[0]) <= 1e-6f);
  // Closed form: logp(4) = 4 - log(e^1 + e^4 + e^2 + e^3 + e^0).
  const double lse = std::log(std::exp(1.0) + std::exp(4.0) + std::exp(2.0) + std::exp(3.0) + 1.0);
  KAT_CHECK(std::fabs(r.logprobs[0] - (4.0 - lse)) <= 1e-5);
}

void case_full_top_k_normalised(Sampler& s) {  // :183-192
  Logits lg({{0.5f, 1.5f, -0.5f, 2.0f}});
  SamplingParams p;
  p.temperature = 0.0f;
  p.top_logprobs = 4;
  SampleResult r = s.sample(lg.view(), p, {0.5f});
  double sum = 0.0;
  for (float x : r.top_logprobs) sum += std::exp(static_cast<double>(x));
  KAT_CHECK(std::fabs(sum - 1.0) <= 1e-5);  // the reference allows 1%
}

void case_top_logprobs_pre_temperature(Sampler& s) {  // :194-203
  Logits lg({{1.0f, 4.0f, 2.0f, 3.0f}});
  SamplingParams p;
  p.temperature = 0.8f;
  p.top_logprobs = 2;
  SampleResult r = s.sample(lg.view(), p, {0.3f});
  KAT_CHECK(r.K == 2);
  KAT_CHECK((r.top_tokens == std::vector<int32_t>{1, 3}));
}

void case_min_p(Sampler& s) {  // :76-87
  // probs [0.5, 0.3, 0.15, 0.05]; min_p 0.4 keeps prob >= 0.2, i.e. {0, 1}
  Logits lg({log_of({0.5f, 0.3f, 0.15f, 0.05f})});
  SamplingParams p;
  p.min_p = 0.4f;
  std::set<int> kept = kept_by_sweep(s, lg, p, 64);
  KAT_CHECK((kept == std::set<int>{0, 1}));
}

// The filter entry points (sampler_test.cpp:54-87 call Sampler::apply_top_k /
// apply_top_p / apply_min_p directly): finite entries after the filter.
std::vector<bool> finite_after(Sampler& s, const std::vector<float>& z, int which, float arg) {
  Logits lg({z});
  float* out = nullptr;
  if (hipMalloc(reinterpret_cast<void**>(&out), z.size() * sizeof(float)) != hipSuccess) std::exit(2);
  if (which == 0) s.apply_top_k(lg.view(), static_cast<int>(arg), out);
  if (which == 1) s.apply_top_p(lg.view(), arg, out);
  if (which == 2) s.apply_min_p(lg.view(), arg, out);
  std::vector<float> h(z.size());
  (void)hipMemcpy(h.data(), out, z.size() * sizeof(float), hipMemcpyDeviceToHost);
  (void)hipFree(out);
  std::vector<bool> f(z.size());
  for (size_t i = 0; i < z.size(); ++i) f[i] = std::isfinite(h[i]) && h[i] == z[i];
  return f;
}

void case_filter_entry_points(Sampler& s) {  // :54-87
  KAT_CHECK((finite_after(s, {5.0f, 1.0f, 4.0f, 2.0f, 3.0f}, 0, 2.0f) ==
             std::vector<bool>{true, false, true, false, false}));
  const std::vector<float> lg = log_of({0.5f, 0.3f, 0.15f, 0.05f});
  KAT_CHECK((finite_after(s, lg, 1, 0.7f) == std::vector<bool>{true, true, false, false}));
  KAT_CHECK((finite_after(s, lg, 2, 0.4f) == std::vector<bool>{true, true, false, false}));
}

void case_penalties_refused(Sampler& s) {  // :89-124 need apply_penalties first
  Logits lg({{2.0f, 1.0f, 0.5f}});
  for (int which = 0; which < 3; ++which) {
    SamplingParams p;
    if (which == 0) p.repetition_penalty = 4.0f;
    if (which == 1) p.frequency_penalty = 0.5f;
    if (which == 2) p.presence_penalty = 0.7f;
    bool threw = false;
    try {
      s.sample(lg.view(), p, {0.5f});
    } catch (const SamplerError& e) {
      threw = e.code() == MLXF_EINVAL;
    }
    KAT_CHECK(threw);
  }
}

std::vector<float> penalized(Sampler& s, const std::vector<float>& z, const std::vector<int32_t>& hist,
                             const SamplingParams& p) {
  Logits lg({z});
  s.apply_penalties(lg.d, MLXF_DTYPE_F32, 1, static_cast<int>(z.size()), 0, {hist}, {p});
  std::vector<float> out(z.size());
  (void)hipMemcpy(out.data(), lg.d, z.size() * sizeof(float), hipMemcpyDeviceToHost);
  return out;
}

void case_repetition_penalty(Sampler& s) {  // :89-98
  SamplingParams p;
  p.repetition_penalty = 4.0f;
  std::vector<float> f = penalized(s, {2.0f, 1.0f, 0.5f}, {0}, p);
  KAT_CHECK(f[0] == 0.5f);  // 2.0 / 4.0
  KAT_CHECK(f[1] == 1.0f);  // untouched
  KAT_CHECK(f[0] < f[1]);
}

void case_frequency_presence(Sampler& s) {  // :100-115
  SamplingParams pf;
  pf.frequency_penalty = 0.5f;
  std::vector<float> f = penalized(s, {0.0f, 0.0f, 0.0f, 0.0f}, {1, 1, 2}, pf);
  KAT_CHECK((f == std::vector<float>{0.0f, -1.0f, -0.5f, 0.0f}));
  SamplingParams pp;
  pp.presence_penalty = 0.7f;
  std::vector<float> g = penalized(s, {0.0f, 0.0f, 0.0f, 0.0f}, {1, 1, 2}, pp);
  KAT_CHECK(g[0] == 0.0f && g[3] == 0.0f);
  KAT_CHECK(g[1] == -0.7f && g[2] == -0.7f);
}

void case_penalty_moves_greedy(Sampler& s) {  // :117-124
  Logits lg({{2.0f, 1.0f, 0.5f}});
  SamplingParams p;
  p.temperature = 0.0f;
  p.repetition_penalty = 4.0f;
  s.apply_penalties(lg.d, MLXF_DTYPE_F32, 1, 3, 0, {{0}}, {p});
  p.repetition_penalty = 1.0f;  // applied
  SampleResult r = s.sample(lg.view(), p, {0.5f});
  KAT_CHECK((r.tokens == std::vector<int32_t>{1}));
}

void case_seeded_uniforms(Sampler&) {  // :126-134 with a seed instead of a key
  // u = Philox4x32-10(key = seed, counter = (step, 0)) word 0 >> 8, * 2^-24:
  // the published vector for key 0, counter 0 starts 0x6627e8d5
  std::vector<uint64_t> seed = {0, 0, 42};
  std::vector<uint64_t> step = {0, 1, 0};
  uint64_t *ds = nullptr, *dt = nullptr;
  float* du = nullptr;
  (void)hipMalloc(reinterpret_cast<void**>(&ds), 3 * sizeof(uint64_t));
  (void)hipMalloc(reinterpret_cast<void**>(&dt), 3 * sizeof(uint64_t));
  (void)hipMalloc(reinterpret_cast<void**>(&du), 3 * sizeof(float));
  (void)hipMemcpy(ds, seed.data(), 3 * sizeof(uint64_t), hipMemcpyHostToDevice);
  (void)hipMemcpy(dt, step.data(), 3 * sizeof(uint64_t), hipMemcpyHostToDevice);
  char* err = nullptr;
  KAT_CHECK(mlxf_uniforms(3, ds, dt, 0, du, nullptr, &err) == MLXF_OK);
  std::vector<float> u(3), u2(3);
  (void)hipMemcpy(u.data(), du, 3 * sizeof(float), hipMemcpyDeviceToHost);
  KAT_CHECK(u[0] == static_cast<float>(0x6627e8d5u >> 8) * 0x1p-24f);
  KAT_CHECK(u[1] != u[0] && u[2] != u[0]);  // another step, another seed
  KAT_CHECK(mlxf_uniforms(3, ds, dt, 0, du, nullptr, &err) == MLXF_OK);
  (void)hipMemcpy(u2.data(), du, 3 * sizeof(float), hipMemcpyDeviceToHost);
  KAT_CHECK(u == u2);  // same seed and step: same uniform
  (void)hipFree(ds);
  (void)hipFree(dt);
  (void)hipFree(du);
}

void case_grammar_mask(Sampler& s) {  // src/runtime/worker.cpp:142-179,455-459
  // only tokens 1 and 3 allowed: greedy picks the best allowed one, and no
  // draw ever returns a forbidden token
  Logits lg({{5.0f, 1.0f, 4.0f, 2.0f, 3.0f}});
  uint32_t bits = (1u << 1) | (1u << 3);
  uint32_t* db = nullptr;
  float* dout = nullptr;
  (void)hipMalloc(reinterpret_cast<void**>(&db), sizeof(uint32_t));
  (void)hipMalloc(reinterpret_cast<void**>(&dout), 5 * sizeof(float));
  (void)hipMemcpy(db, &bits, sizeof(uint32_t), hipMemcpyHostToDevice);
  char* err = nullptr;
  KAT_CHECK(mlxf_apply_mask(lg.d, MLXF_DTYPE_F32, 1, 5, 5, db, 1, dout, 5, nullptr, &err) == MLXF_OK);
  std::vector<float> m(5);
  (void)hipMemcpy(m.data(), dout, 5 * sizeof(float), hipMemcpyDeviceToHost);
  KAT_CHECK(m[1] == 1.0f && m[3] == 2.0f);
  KAT_CHECK(std::isinf(m[0]) && m[0] < 0 && std::isinf(m[2]) && std::isinf(m[4]));
  DeviceLogits v{dout, MLXF_DTYPE_F32, 1, 5, 0};
  KAT_CHECK((s.greedy(v) == std::vector<int32_t>{3}));
  SamplingParams p;
  std::set<int> seen;
  for (int i = 0; i < 32; ++i) seen.insert(s.sample_rows(v, {p}, {(i + 0.5f) / 32.0f}).tokens[0]);
  KAT_CHECK((seen == std::set<int>{1, 3}));
  // nothing allowed: the row is left as it is (the reference adds zeros)
  bits = 0u;
  (void)hipMemcpy(db, &bits, sizeof(uint32_t), hipMemcpyHostToDevice);
  KAT_CHECK(mlxf_apply_mask(lg.d, MLXF_DTYPE_F32, 1, 5, 5, db, 1, dout, 5, nullptr, &err) == MLXF_OK);
  KAT_CHECK((s.greedy(v) == std::vector<int32_t>{0}));
  (void)hipFree(db);
  (void)hipFree(dout);
}

void case_row_stride(Sampler& s) {  // the (bucket, 1, V) view with B rows sampled
  // Rows of 5 logits inside rows of 8; the padding holds a value that would win.
  Logits lg({{0.0f, 1.0f, 3.0f, 2.0f, 0.5f, 99.0f, 99.0f, 99.0f},
             {4.0f, 1.0f, 3.0f, 2.0f, 0.5f, 99.0f, 99.0f, 99.0f}});
  DeviceLogits v{lg.d, MLXF_DTYPE_F32, 2, 5, 8};
  KAT_CHECK((s.greedy(v) == std::vector<int32_t>{2, 0}));
}

void case_error_reporting(Sampler& s) {  // errors cross the ABI as codes + messages
  Logits lg({{1.0f, 2.0f}});
  DeviceLogits v = lg.view();
  v.dtype = 7;
  bool threw = false;
  try {
    s.greedy(v);
  } catch (const SamplerError& e) {
    threw = e.code() == MLXF_EINVAL && std::string(e.what()).size() > 0;
  }
  KAT_CHECK(threw);
}

}  // namespace

int main() {
  int ndev = 0;
  if (hipGetDeviceCount(&ndev) != hipSuccess || ndev < 1) {
    std::fprintf(stderr, "sampler_kat: no GPU\n");
    return 2;
  }
  hipStream_t st;
  if (hipStreamCreate(&st) != hipSuccess) return 2;
  struct Case {
    const char* name;
    void (*fn)(Sampler&);
  } cases[] = {
      {"greedy returns the argmax index", case_greedy},
      {"temperature 0 collapses to greedy", case_temperature_zero},
      {"top-k keeps exactly k candidates", case_top_k},
      {"top-p keeps the smallest prefix whose mass >= p", case_top_p},
      {"same uniforms reproduce, different uniforms diverge", case_reproducible},
      {"sample returns batched tokens and logprobs", case_batched},
      {"top_logprobs off leaves the top arrays empty", case_top_logprobs_off},
      {"top_logprobs == 0 reports the chosen logprob only", case_top_logprobs_zero},
      {"top_logprobs > 0 ranks ids by descending logprob", case_top_logprobs_ranked},
      {"a full top-k recovers a normalised distribution", case_full_top_k_normalised},
      {"top_logprobs come from the pre-temperature logits", case_top_logprobs_pre_temperature},
      {"min-p keeps tokens with prob >= min_p * max_prob", case_min_p},
      {"apply_top_k / apply_top_p / apply_min_p on the reference's cases", case_filter_entry_points},
      {"penalties left in the parameters are refused", case_penalties_refused},
      {"repetition penalty pushes a seen token below an unseen one", case_repetition_penalty},
      {"frequency penalty scales with count, presence is flat", case_frequency_presence},
      {"repetition penalty changes greedy choice", case_penalty_moves_greedy},
      {"same seed and step give the same uniform (device Philox)", case_seeded_uniforms},
      {"the grammar mask only lets allowed tokens through", case_grammar_mask},
      {"row_stride samples B rows of a padded buffer", case_row_stride},
      {"errors carry a code and a message", case_error_reporting},
  };
  try {
    Sampler s(st);
    for (const Case& c : cases) {
      const int before = g_failures;
      c.fn(s);
      std::printf("%s: %s\n", g_failures == before ? "ok  " : "FAIL", c.name);
      std::fflush(stdout);
    }
  } catch (const std::exception& e) {
    std::fprintf(stderr, "sampler_kat: unexpected exception: %s\n", e.what());
    return 1;
  }
  (void)hipStreamDestroy(st);
  std::printf("%d checks, %d failed\n", g_checks, g_failures);
  return g_failures == 0 ? 0 : 1;
}
