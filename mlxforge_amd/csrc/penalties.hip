// penalties.hip -- repetition / frequency / presence penalties on the logits,
// in place, before sampling: the `adj` of Sampler::sample
// (src/sample/sampler.cpp:122-133, applied at :144 when a row has penalties
// and a non-empty history, src/runtime/worker.cpp:469-472).
//
// Two launches over the history entries of every row:
//   k_pen_count  adds 1 to cnt[r][id] for each history id (device atomics);
//   k_pen_apply  takes cnt[r][id] with an atomic exchange against 0: exactly
//                one entry per distinct id gets the total count and updates
//                that logit; every counter is back to 0 afterwards, so the
//                counter array (caller-owned, zeroed once) is ready for the
//                next call.
// The update follows the reference's graph ops, each rounded to the logits
// dtype: repetition z > 0 ? z / pen : z * pen (src/sample/sampler.cpp:95-105),
// then z - count * frequency - presence (:107-120), with pen, frequency,
// presence and the count as values of the logits dtype.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <string>

#include "device_common.hpp"
#include "mlxf_sampler.h"

namespace mlxf {
namespace {

constexpr int PEN_THREADS = 256;

struct PenArgs {
  void* logits;
  long long row_stride;
  int B, V;
  const int* hist;
  long long hist_stride;
  const int* hist_len;
  const float* rep;
  const float* freq;
  const float* pres;
  unsigned int* cnt;  // [B][V]
};

struct PenRow {
  float rep, freq, pres;
  bool on;
};

// The C ABI's sanitisation (src/capi/mlxforge.cpp:59-64): a repetition
// penalty that is not finite and positive is 1 (off); a frequency or presence
// penalty that is not finite is 0 (off).
__device__ __forceinline__ PenRow pen_row(const PenArgs& a, int r) {
  PenRow p;
  const float rp = a.rep ? a.rep[r] : 1.0f;
  const float fq = a.freq ? a.freq[r] : 0.0f;
  const float ps = a.pres ? a.pres[r] : 0.0f;
  p.rep = (__builtin_isfinite(rp) && rp > 0.0f) ? rp : 1.0f;
  p.freq = __builtin_isfinite(fq) ? fq : 0.0f;
  p.pres = __builtin_isfinite(ps) ? ps : 0.0f;
  p.on = p.rep != 1.0f || p.freq != 0.0f || p.pres != 0.0f;
  return p;
}

template <int DT>
__device__ __forceinline__ float ld_logit(const void* row, int i) {
  if constexpr (DT == MLXF_DTYPE_F32) {
    return static_cast<const float*>(row)[i];
  } else if constexpr (DT == MLXF_DTYPE_BF16) {
    return __uint_as_float(static_cast<unsigned int>(static_cast<const unsigned short*>(row)[i]) << 16);
  } else {
    return __half2float(static_cast<const __half*>(row)[i]);
  }
}

// x is a value of the logits dtype (the rounding of the last step).
template <int DT>
__device__ __forceinline__ void st_logit(void* row, int i, float x) {
  if constexpr (DT == MLXF_DTYPE_F32) {
    static_cast<float*>(row)[i] = x;
  } else if constexpr (DT == MLXF_DTYPE_BF16) {
    static_cast<unsigned short*>(row)[i] = static_cast<unsigned short>(__float_as_uint(x) >> 16);
  } else {
    static_cast<__half*>(row)[i] = __float2half_rn(x);
  }
}

__device__ __forceinline__ int hist_len(const PenArgs& a, int r) {
  const int n = a.hist_len ? a.hist_len[r] : static_cast<int>(a.hist_stride);
  return n < 0 ? 0 : (n > a.hist_stride ? static_cast<int>(a.hist_stride) : n);
}

// grid (ceil(max history / PEN_THREADS), B)
__global__ __launch_bounds__(PEN_THREADS) void k_pen_count(PenArgs a) {
  const int r = static_cast<int>(blockIdx.y);
  const int j = static_cast<int>(blockIdx.x) * PEN_THREADS + static_cast<int>(threadIdx.x);
  if (j >= hist_len(a, r) || !pen_row(a, r).on) return;
  const int id = a.hist[static_cast<size_t>(r) * a.hist_stride + j];
  if (id < 0 || id >= a.V) return;
  __hip_atomic_fetch_add(a.cnt + static_cast<size_t>(r) * a.V + id, 1u, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
}

template <int DT>
__global__ __launch_bounds__(PEN_THREADS) void k_pen_apply(PenArgs a) {
  const int r = static_cast<int>(blockIdx.y);
  const int j = static_cast<int>(blockIdx.x) * PEN_THREADS + static_cast<int>(threadIdx.x);
  if (j >= hist_len(a, r)) return;
  const PenRow p = pen_row(a, r);
  if (!p.on) return;
  const int id = a.hist[static_cast<size_t>(r) * a.hist_stride + j];
  if (id < 0 || id >= a.V) return;
  const unsigned int c = __hip_atomic_exchange(a.cnt + static_cast<size_t>(r) * a.V + id, 0u,
                                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (c == 0u) return;  // another entry of the same id took the count
  void* row = static_cast<char*>(a.logits) +
              static_cast<size_t>(r) * static_cast<size_t>(a.row_stride) * elem_size<DT>();
  float z = ld_logit<DT>(row, id);
  if (z != z) return;  // NaN stays NaN (the sampler reads it as -inf)
  if (p.rep != 1.0f) {
    const float pen = round_dt<DT>(p.rep);
    z = z > 0.0f ? round_dt<DT>(z / pen) : round_dt<DT>(z * pen);
  }
  if (p.freq != 0.0f || p.pres != 0.0f) {
    const float cd = round_dt<DT>(static_cast<float>(c));
    z = round_dt<DT>(z - round_dt<DT>(cd * round_dt<DT>(p.freq)));
    z = round_dt<DT>(z - round_dt<DT>(p.pres));
  }
  st_logit<DT>(row, id, z);
}

void set_err(char** err, const std::string& msg) {
  if (!err) return;
  char* q = static_cast<char*>(std::malloc(msg.size() + 1));
  if (q) std::memcpy(q, msg.c_str(), msg.size() + 1);
  *err = q;
}

}  // namespace
}  // namespace mlxf

extern "C" {

int mlxf_penalties_workspace_size(int B, int V, size_t* bytes, char** err) {
  if (B < 0 || V < 1 || V > MLXF_MAX_VOCAB || !bytes) {
    mlxf::set_err(err, "mlxf: penalties workspace needs B >= 0, V in [1, MLXF_MAX_VOCAB] and bytes");
    return MLXF_EINVAL;
  }
  *bytes = (static_cast<size_t>(B > 0 ? B : 1) * static_cast<size_t>(V) * sizeof(unsigned int) + 255) &
           ~static_cast<size_t>(255);
  return MLXF_OK;
}

int mlxf_apply_penalties(void* d_logits, int dtype, int B, int V, int64_t row_stride,
                         const int32_t* d_history, int64_t hist_stride, const int32_t* d_hist_len,
                         const float* d_repetition, const float* d_frequency, const float* d_presence,
                         void* d_workspace, size_t workspace_bytes, void* stream, char** err) {
  using namespace mlxf;
  if (dtype != MLXF_DTYPE_F32 && dtype != MLXF_DTYPE_BF16 && dtype != MLXF_DTYPE_F16) {
    set_err(err, "mlxf: dtype must be MLXF_DTYPE_F32, MLXF_DTYPE_BF16 or MLXF_DTYPE_F16");
    return MLXF_EINVAL;
  }
  if (B < 0 || B > 65535 || V < 1 || V > MLXF_MAX_VOCAB || row_stride < V || hist_stride < 0 ||
      hist_stride > (int64_t{1} << 30)) {
    set_err(err, "mlxf: bad shape (B in [0, 65535], V in [1, MLXF_MAX_VOCAB], row_stride >= V, "
                 "0 <= hist_stride <= 2^30)");
    return MLXF_EINVAL;
  }
  if (B == 0 || hist_stride == 0 || (!d_repetition && !d_frequency && !d_presence)) return MLXF_OK;
  if (!d_logits || !d_history) {
    set_err(err, "mlxf: d_logits and d_history must not be NULL");
    return MLXF_EINVAL;
  }
  size_t need = 0;
  mlxf_penalties_workspace_size(B, V, &need, nullptr);
  if (!d_workspace || workspace_bytes < need) {
    set_err(err, "mlxf: workspace is NULL or smaller than mlxf_penalties_workspace_size()");
    return MLXF_EWORKSPACE;
  }
  const size_t esz = dtype == MLXF_DTYPE_F32 ? 4 : 2;
  if (reinterpret_cast<uintptr_t>(d_logits) % esz || reinterpret_cast<uintptr_t>(d_workspace) % 4) {
    set_err(err, "mlxf: d_logits or the workspace is misaligned");
    return MLXF_EINVAL;
  }
  PenArgs a;
  a.logits = d_logits;
  a.row_stride = row_stride;
  a.B = B;
  a.V = V;
  a.hist = d_history;
  a.hist_stride = hist_stride;
  a.hist_len = d_hist_len;
  a.rep = d_repetition;
  a.freq = d_frequency;
  a.pres = d_presence;
  a.cnt = static_cast<unsigned int*>(d_workspace);
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned int>((hist_stride + PEN_THREADS - 1) / PEN_THREADS),
                  static_cast<unsigned int>(B));
  hipLaunchKernelGGL(k_pen_count, grid, dim3(PEN_THREADS), 0, st, a);
  if (dtype == MLXF_DTYPE_F32)
    hipLaunchKernelGGL(k_pen_apply<MLXF_DTYPE_F32>, grid, dim3(PEN_THREADS), 0, st, a);
  else if (dtype == MLXF_DTYPE_BF16)
    hipLaunchKernelGGL(k_pen_apply<MLXF_DTYPE_BF16>, grid, dim3(PEN_THREADS), 0, st, a);
  else
    hipLaunchKernelGGL(k_pen_apply<MLXF_DTYPE_F16>, grid, dim3(PEN_THREADS), 0, st, a);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_err(err, std::string("mlxf: kernel launch failed: ") + hipGetErrorString(e));
    return MLXF_EHIP;
  }
  return MLXF_OK;
}

}  // extern "C"
