// sampler.hpp -- C++ host wrapper over the C ABI of libmlxf_sampler
// (include/mlxf_sampler.h), mirroring the reference's sampler interface
// (src/sample/sampler.h:15-79) for C++ callers such as a decode-step worker.
//
//   mlxforge::SamplingParams / SampleResult / Sampler  (src/sample/sampler.h)
//   ->  mlxforge_amd::SamplingParams / SampleResult / Sampler
//
// Differences the boundary forces, each stated where it appears:
//   * logits are a device view (DeviceLogits) instead of an mx::array;
//   * the MLX PRNG key is replaced by one caller-supplied uniform per row
//     (inverse-CDF draw; the reference's random::categorical,
//     src/sample/sampler.cpp:165);
//   * results are copied back to host vectors (what the reference's worker
//     does right after its async_eval, src/runtime/worker.cpp:498-512);
//   * the penalties are applied to the logits beforehand (apply_penalties on
//     a mutable view; the reference builds a penalized copy, `adj`,
//     src/sample/sampler.cpp:144): sample() reports penalties left in its
//     params as an error instead of ignoring them.
// Header-only; needs the HIP runtime for device buffers and copies.  The
// sampler library itself never allocates: this wrapper owns the workspace.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <stdexcept>
#include <string>
#include <vector>

#include "mlxf_sampler.h"

namespace mlxforge_amd {

// src/sample/sampler.h:15-36, same fields, defaults and sentinels.
struct SamplingParams {
  float temperature = 1.0f;  // <= 0 => greedy (argmax)
  int top_k = 0;             // <= 0 => disabled
  float top_p = 1.0f;        // >= 1 => disabled
  float min_p = 0.0f;        // <= 0 => disabled; applied after top-p
  float repetition_penalty = 1.0f;
  float frequency_penalty = 0.0f;
  float presence_penalty = 0.0f;
  uint64_t seed = 0;
  int top_logprobs = -1;  // -1 off, 0 chosen only, N > 0 alternatives

  bool has_penalties() const {
    return repetition_penalty != 1.0f || frequency_penalty != 0.0f || presence_penalty != 0.0f;
  }
};

// src/sample/sampler.h:38-45 as host vectors; top_* are row-major (B, K).
struct SampleResult {
  std::vector<int32_t> tokens;
  std::vector<float> logprobs;
  int K = 0;
  std::vector<int32_t> top_tokens;
  std::vector<float> top_logprobs;
};

// A [B, V] logits matrix in device memory; row r starts at data + r * row_stride.
struct DeviceLogits {
  const void* data = nullptr;
  int dtype = MLXF_DTYPE_F32;
  int B = 0;
  int V = 0;
  int64_t row_stride = 0;  // 0: V
};

class SamplerError : public std::runtime_error {
 public:
  SamplerError(int code, const std::string& msg) : std::runtime_error(msg), code_(code) {}
  int code() const { return code_; }

 private:
  int code_;
};

namespace detail {
inline void check(int rc, char* err) {
  if (rc == MLXF_OK) return;
  std::string msg = err ? err : "mlxf: error";
  mlxf_string_free(err);
  throw SamplerError(rc, msg);
}
inline void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) throw SamplerError(MLXF_EHIP, std::string(what) + ": " + hipGetErrorString(e));
}
template <typename T>
struct DeviceBuf {
  T* p = nullptr;
  size_t n = 0;
  void reserve(size_t want) {
    if (want <= n) return;
    if (p) (void)hipFree(p);
    p = nullptr;
    n = 0;
    hip_check(hipMalloc(reinterpret_cast<void**>(&p), want * sizeof(T) + 256), "hipMalloc");
    n = want;
  }
  ~DeviceBuf() {
    if (p) (void)hipFree(p);
  }
};
// Page-locked host staging (hipHostMalloc), so the one upload and the one
// readback of a step are true asynchronous copies.
struct PinnedBuf {
  unsigned char* p = nullptr;
  size_t n = 0;
  void reserve(size_t want) {
    if (want <= n) return;
    if (p) (void)hipHostFree(p);
    p = nullptr;
    n = 0;
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&p), want, hipHostMallocDefault), "hipHostMalloc");
    n = want;
  }
  ~PinnedBuf() {
    if (p) (void)hipHostFree(p);
  }
};
inline size_t align64(size_t x) { return (x + 63) & ~static_cast<size_t>(63); }
}  // namespace detail

// Batched sampler on one HIP stream.  Reuses its device buffers across calls;
// not thread-safe (one instance per worker thread / stream, as the reference
// confines MLX to its worker thread, src/runtime/worker.h:1-4).
class Sampler {
 public:
  explicit Sampler(hipStream_t stream = nullptr) : stream_(stream) {}
  Sampler(const Sampler&) = delete;
  Sampler& operator=(const Sampler&) = delete;

  // One token per row with per-row parameters: what Worker::sample_rows +
  // finalize_sample compute (src/runtime/worker.cpp:448-514), in one launch.
  SampleResult sample_rows(const DeviceLogits& logits, const std::vector<SamplingParams>& params,
                           const std::vector<float>& uniforms) {
    const int B = logits.B;
    if (static_cast<int>(params.size()) != B || static_cast<int>(uniforms.size()) != B)
      throw SamplerError(MLXF_EINVAL, "mlxf: params and uniforms need one entry per row");
    std::vector<float> T(B), p(B), mp(B);
    std::vector<int32_t> k(B), tlp(B);
    int K_max = 0;
    for (int r = 0; r < B; ++r) {
      const SamplingParams& sp = params[r];
      if (sp.has_penalties())
        throw SamplerError(MLXF_EINVAL, "mlxf: penalties must be applied to the logits first");
      T[r] = sp.temperature;
      k[r] = sp.top_k;
      p[r] = sp.top_p;
      mp[r] = sp.min_p;
      tlp[r] = sp.top_logprobs;
      if (sp.top_logprobs > K_max) K_max = sp.top_logprobs;
    }
    if (K_max > logits.V) K_max = logits.V;
    if (K_max > MLXF_MAX_TOP_LOGPROBS)
      throw SamplerError(MLXF_EINVAL, "mlxf: top_logprobs above MLXF_MAX_TOP_LOGPROBS");
    return run(logits, T.data(), k.data(), p.data(), mp.data(), tlp.data(), uniforms.data(), K_max);
  }

  // Sampler::sample(logits, params, key) (src/sample/sampler.h:51-52) with one
  // parameter set for every row.  As in the reference, the chosen-token
  // logprob is always computed (src/sample/sampler.cpp:151-154).
  SampleResult sample(const DeviceLogits& logits, const SamplingParams& params,
                      const std::vector<float>& uniforms) {
    std::vector<SamplingParams> rows(logits.B, params);
    for (auto& r : rows) r.top_logprobs = params.top_logprobs < 0 ? 0 : params.top_logprobs;
    return sample_rows(logits, rows, uniforms);
  }

  // The penalized `adj` of Sampler::sample (src/sample/sampler.cpp:95-133,144),
  // written over the logits in place: row r of `history` holds its token ids
  // (prompt and generated so far, src/runtime/worker.cpp:415,437,549); each
  // row's penalties come from its SamplingParams.  Call before sample_rows on
  // the same logits; sample_rows then needs the penalties cleared from params.
  void apply_penalties(void* logits, int dtype, int B, int V, int64_t row_stride,
                       const std::vector<std::vector<int32_t>>& history,
                       const std::vector<SamplingParams>& params) {
    if (static_cast<int>(history.size()) != B || static_cast<int>(params.size()) != B)
      throw SamplerError(MLXF_EINVAL, "mlxf: history and params need one entry per row");
    size_t N = 0;
    for (const auto& h : history) N = h.size() > N ? h.size() : N;
    if (B == 0 || N == 0) return;
    std::vector<int32_t> flat(static_cast<size_t>(B) * N, 0), len(B);
    std::vector<float> rep(B), fq(B), ps(B);
    for (int r = 0; r < B; ++r) {
      std::copy(history[r].begin(), history[r].end(), flat.begin() + static_cast<size_t>(r) * N);
      len[r] = static_cast<int32_t>(history[r].size());
      rep[r] = params[r].repetition_penalty;
      fq[r] = params[r].frequency_penalty;
      ps[r] = params[r].presence_penalty;
    }
    char* err = nullptr;
    size_t pw = 0;
    detail::check(mlxf_penalties_workspace_size(B, V, &pw, &err), err);
    if (pw > pen_ws_bytes_) {
      pen_ws_.reserve(pw);
      pen_ws_bytes_ = pw;
      // once per growth, outside any steady-state step: the counters start at
      // zero and every call leaves them there
      detail::hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
      detail::hip_check(hipMemset(pen_ws_.p, 0, pw), "hipMemset");
    }
    upload(hist_, flat.data(), static_cast<int>(flat.size()));
    upload(hlen_, len.data(), B);
    upload(rep_, rep.data(), B);
    upload(fq_, fq.data(), B);
    upload(ps_, ps.data(), B);
    err = nullptr;
    detail::check(mlxf_apply_penalties(logits, dtype, B, V, row_stride ? row_stride : V, hist_.p,
                                       static_cast<int64_t>(N), hlen_.p, rep_.p, fq_.p, ps_.p, pen_ws_.p,
                                       pen_ws_bytes_, stream_, &err),
                  err);
  }

  // Sampler::apply_top_k / apply_top_p / apply_min_p (src/sample/sampler.h:63-69):
  // the logits with every removed entry set to -inf, written to d_out (the
  // logits' dtype, row stride out_stride, 0: V; d_out may be logits.data for
  // in place).  Asynchronous on the sampler's stream.
  void apply_top_k(const DeviceLogits& logits, int k, void* d_out, int64_t out_stride = 0) {
    char* err = nullptr;
    ensure_filter_workspace(logits);
    detail::check(mlxf_apply_top_k(logits.data, logits.dtype, logits.B, logits.V, stride_of(logits), k, d_out,
                                   out_stride ? out_stride : logits.V, flt_ws_.p, flt_ws_bytes_, stream_, &err),
                  err);
  }
  void apply_top_p(const DeviceLogits& logits, float p, void* d_out, int64_t out_stride = 0) {
    char* err = nullptr;
    ensure_filter_workspace(logits);
    detail::check(mlxf_apply_top_p(logits.data, logits.dtype, logits.B, logits.V, stride_of(logits), p, d_out,
                                   out_stride ? out_stride : logits.V, flt_ws_.p, flt_ws_bytes_, stream_, &err),
                  err);
  }
  void apply_min_p(const DeviceLogits& logits, float min_p, void* d_out, int64_t out_stride = 0) {
    char* err = nullptr;
    ensure_filter_workspace(logits);
    detail::check(mlxf_apply_min_p(logits.data, logits.dtype, logits.B, logits.V, stride_of(logits), min_p, d_out,
                                   out_stride ? out_stride : logits.V, flt_ws_.p, flt_ws_bytes_, stream_, &err),
                  err);
  }

  // Sampler::greedy (src/sample/sampler.h:61): argmax, lowest index on ties.
  std::vector<int32_t> greedy(const DeviceLogits& logits) {
    const int B = logits.B, V = logits.V;
    const int64_t stride = logits.row_stride ? logits.row_stride : V;
    char* err = nullptr;
    size_t ws = 0;
    detail::check(mlxf_sampler_workspace_size(B, V, 0, logits.dtype, &ws, &err), err);
    ensure_workspace(ws);
    ids_.reserve(B > 0 ? B : 1);
    err = nullptr;
    detail::check(mlxf_greedy(logits.data, logits.dtype, B, V, stride, ids_.p, ws_.p, ws_bytes_,
                              stream_, &err),
                  err);
    std::vector<int32_t> out(B);
    if (B) {
      detail::hip_check(hipMemcpyAsync(out.data(), ids_.p, B * sizeof(int32_t), hipMemcpyDeviceToHost, stream_),
                        "hipMemcpyAsync");
    }
    detail::hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    return out;
  }

 private:
  static int64_t stride_of(const DeviceLogits& l) { return l.row_stride ? l.row_stride : l.V; }
  void ensure_filter_workspace(const DeviceLogits& logits) {
    size_t need = 0;
    char* err = nullptr;
    detail::check(mlxf_filter_workspace_size(logits.B, logits.V, &need, &err), err);
    if (need > flt_ws_bytes_) {
      flt_ws_.reserve(need);
      flt_ws_bytes_ = need;
    }
  }
  void ensure_workspace(size_t bytes) {
    if (bytes <= ws_bytes_) return;
    ws_.reserve(bytes);
    ws_bytes_ = bytes;
    char* err = nullptr;
    detail::check(mlxf_sampler_workspace_init(ws_.p, ws_bytes_, stream_, &err), err);
  }

  template <typename T>
  void upload(detail::DeviceBuf<T>& d, const T* h, int n) {
    d.reserve(n > 0 ? n : 1);
    if (n)
      detail::hip_check(hipMemcpyAsync(d.p, h, n * sizeof(T), hipMemcpyHostToDevice, stream_),
                        "hipMemcpyAsync");
  }

  // One step: the six per-row parameter arrays go up in one copy from a
  // packed pinned buffer, and ids, logprobs and the top-K block come back in
  // one copy into another (the reference's worker reads its results back
  // once per step, src/runtime/worker.cpp:488-514).
  SampleResult run(const DeviceLogits& logits, const float* T, const int32_t* k, const float* p,
                   const float* mp, const int32_t* tlp, const float* u, int K_max) {
    const int B = logits.B, V = logits.V;
    const int64_t stride = logits.row_stride ? logits.row_stride : V;
    char* err = nullptr;
    size_t ws = 0;
    detail::check(mlxf_sampler_workspace_size(B, V, K_max, logits.dtype, &ws, &err), err);
    ensure_workspace(ws);
    SampleResult res;
    res.K = K_max;
    res.tokens.resize(B);
    res.logprobs.resize(B);
    const size_t BK = static_cast<size_t>(B) * K_max;
    res.top_tokens.resize(BK);
    res.top_logprobs.resize(BK);
    if (B == 0) return res;
    // parameters: T, k, p, min_p, top_logprobs, u (4 bytes each per row)
    const size_t col = detail::align64(static_cast<size_t>(B) * 4);
    const size_t in_bytes = 6 * col;
    in_h_.reserve(in_bytes);
    in_d_.reserve(in_bytes);
    unsigned char* h = in_h_.p;
    std::copy(T, T + B, reinterpret_cast<float*>(h + 0 * col));
    std::copy(k, k + B, reinterpret_cast<int32_t*>(h + 1 * col));
    std::copy(p, p + B, reinterpret_cast<float*>(h + 2 * col));
    std::copy(mp, mp + B, reinterpret_cast<float*>(h + 3 * col));
    std::copy(tlp, tlp + B, reinterpret_cast<int32_t*>(h + 4 * col));
    std::copy(u, u + B, reinterpret_cast<float*>(h + 5 * col));
    detail::hip_check(hipMemcpyAsync(in_d_.p, h, in_bytes, hipMemcpyHostToDevice, stream_), "hipMemcpyAsync");
    const unsigned char* d = in_d_.p;
    // results: ids, logprobs, then the (B, K) top ids and logprobs
    const size_t tcol = detail::align64(BK * 4);
    const size_t out_bytes = 2 * col + 2 * tcol;
    out_h_.reserve(out_bytes);
    out_d_.reserve(out_bytes);
    unsigned char* o = out_d_.p;
    // the parameters are on the host here, so only the refine stages some row
    // can need are launched
    const int stages = mlxf_sampler_refine_stages(B, V, logits.dtype, T, k, p);
    err = nullptr;
    detail::check(
        mlxf_sample_ex(logits.data, logits.dtype, B, V, stride, reinterpret_cast<const float*>(d + 0 * col),
                       reinterpret_cast<const int32_t*>(d + 1 * col), reinterpret_cast<const float*>(d + 2 * col),
                       reinterpret_cast<const float*>(d + 3 * col), reinterpret_cast<const int32_t*>(d + 4 * col),
                       reinterpret_cast<const float*>(d + 5 * col), reinterpret_cast<int32_t*>(o),
                       reinterpret_cast<float*>(o + col), K_max ? reinterpret_cast<int32_t*>(o + 2 * col) : nullptr,
                       K_max ? reinterpret_cast<float*>(o + 2 * col + tcol) : nullptr, K_max, ws_.p, ws_bytes_,
                       stages, stream_, &err),
        err);
    detail::hip_check(hipMemcpyAsync(out_h_.p, o, out_bytes, hipMemcpyDeviceToHost, stream_), "hipMemcpyAsync");
    detail::hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
    const unsigned char* q = out_h_.p;
    std::copy(reinterpret_cast<const int32_t*>(q), reinterpret_cast<const int32_t*>(q) + B, res.tokens.begin());
    std::copy(reinterpret_cast<const float*>(q + col), reinterpret_cast<const float*>(q + col) + B,
              res.logprobs.begin());
    if (K_max) {
      std::copy(reinterpret_cast<const int32_t*>(q + 2 * col), reinterpret_cast<const int32_t*>(q + 2 * col) + BK,
                res.top_tokens.begin());
      std::copy(reinterpret_cast<const float*>(q + 2 * col + tcol),
                reinterpret_cast<const float*>(q + 2 * col + tcol) + BK, res.top_logprobs.begin());
    }
    return res;
  }

  hipStream_t stream_;
  detail::DeviceBuf<unsigned char> ws_;
  size_t ws_bytes_ = 0;
  detail::DeviceBuf<unsigned char> in_d_, out_d_;  // packed parameters / results of a step
  detail::PinnedBuf in_h_, out_h_;                  // ... their host staging
  detail::DeviceBuf<float> rep_, fq_, ps_;
  detail::DeviceBuf<int32_t> ids_, hist_, hlen_;
  detail::DeviceBuf<unsigned char> pen_ws_;
  size_t pen_ws_bytes_ = 0;
  detail::DeviceBuf<unsigned char> flt_ws_;  // the filter calls' scratch
  size_t flt_ws_bytes_ = 0;
};

}  // namespace mlxforge_amd
