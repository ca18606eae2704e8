// mask.hip -- the grammar-constrained row of the decode step: logits plus an
// additive fp32 mask of 0 (allowed) / -inf (disallowed), which MLX evaluates
// as an fp32 row (src/runtime/worker.cpp:455-459, the mask built at :142-179).
// Here the mask arrives as one bit per token (1 = allowed), 1/32 of the fp32
// array, and the kernel writes the fp32 row: the logit where allowed, -inf
// elsewhere -- the exact value of row + mask.  A row with no allowed token is
// copied unmasked: the reference never builds an all -inf mask and adds zeros
// instead (:175-177).  The masked rows are then sampled as fp32 logits.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <string>

#include "device_common.hpp"
#include "mlxf_sampler.h"

namespace mlxf {
namespace {

constexpr int MASK_THREADS = 256;

template <int DT>
__global__ __launch_bounds__(MASK_THREADS) void k_mask(const void* logits, long long row_stride, int V,
                                                       const unsigned int* bits, long long bits_stride,
                                                       float* out, long long out_stride) {
  __shared__ int any[WAVES];
  const int r = static_cast<int>(blockIdx.x);
  const int tid = static_cast<int>(threadIdx.x), lane = tid & 63, wid = tid >> 6;
  const unsigned int* b = bits + static_cast<size_t>(r) * static_cast<size_t>(bits_stride);
  const int nw = (V + 31) / 32;
  // any allowed token in the row? (bits past V do not count)
  unsigned int acc = 0u;
  for (int w = tid; w < nw; w += MASK_THREADS) {
    unsigned int x = b[w];
    if (w == nw - 1 && (V & 31)) x &= (1u << (V & 31)) - 1u;
    acc |= x;
  }
  const bool wa = __builtin_amdgcn_ballot_w64(acc != 0u) != 0ull;
  if (lane == 0) any[wid] = wa ? 1 : 0;
  __syncthreads();
  bool allowed_any = false;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) allowed_any |= any[w] != 0;
  const char* row = static_cast<const char*>(logits) + static_cast<size_t>(r) * static_cast<size_t>(row_stride) * elem_size<DT>();
  float* o = out + static_cast<size_t>(r) * static_cast<size_t>(out_stride);
  for (int i = tid; i < V; i += MASK_THREADS) {
    float z;
    if constexpr (DT == MLXF_DTYPE_F32) {
      z = reinterpret_cast<const float*>(row)[i];
    } else if constexpr (DT == MLXF_DTYPE_BF16) {
      z = __uint_as_float(static_cast<unsigned int>(reinterpret_cast<const unsigned short*>(row)[i]) << 16);
    } else {
      z = __half2float(reinterpret_cast<const __half*>(row)[i]);
    }
    const bool ok = !allowed_any || ((b[i >> 5] >> (i & 31)) & 1u);
    o[i] = ok ? z : -INFINITY;
  }
}

void set_err(char** err, const std::string& msg) {
  if (!err) return;
  char* q = static_cast<char*>(std::malloc(msg.size() + 1));
  if (q) std::memcpy(q, msg.c_str(), msg.size() + 1);
  *err = q;
}

}  // namespace
}  // namespace mlxf

extern "C" int mlxf_apply_mask(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                               const uint32_t* d_allowed_bits, int64_t bits_stride, float* d_out,
                               int64_t out_stride, void* stream, char** err) {
  using namespace mlxf;
  if (dtype != MLXF_DTYPE_F32 && dtype != MLXF_DTYPE_BF16 && dtype != MLXF_DTYPE_F16) {
    set_err(err, "mlxf: dtype must be MLXF_DTYPE_F32, MLXF_DTYPE_BF16 or MLXF_DTYPE_F16");
    return MLXF_EINVAL;
  }
  if (B < 0 || V < 1 || V > MLXF_MAX_VOCAB || row_stride < V || out_stride < V ||
      bits_stride < (V + 31) / 32) {
    set_err(err, "mlxf: bad shape (V in [1, MLXF_MAX_VOCAB], row_stride and out_stride >= V, "
                 "bits_stride >= ceil(V / 32))");
    return MLXF_EINVAL;
  }
  if (B == 0) return MLXF_OK;
  if (!d_logits || !d_allowed_bits || !d_out) {
    set_err(err, "mlxf: d_logits, d_allowed_bits and d_out must not be NULL");
    return MLXF_EINVAL;
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned int>(B));
  const unsigned int* bits = reinterpret_cast<const unsigned int*>(d_allowed_bits);
  if (dtype == MLXF_DTYPE_F32)
    hipLaunchKernelGGL(k_mask<MLXF_DTYPE_F32>, grid, dim3(MASK_THREADS), 0, st, d_logits, row_stride, V, bits,
                       bits_stride, d_out, out_stride);
  else if (dtype == MLXF_DTYPE_BF16)
    hipLaunchKernelGGL(k_mask<MLXF_DTYPE_BF16>, grid, dim3(MASK_THREADS), 0, st, d_logits, row_stride, V, bits,
                       bits_stride, d_out, out_stride);
  else
    hipLaunchKernelGGL(k_mask<MLXF_DTYPE_F16>, grid, dim3(MASK_THREADS), 0, st, d_logits, row_stride, V, bits,
                       bits_stride, d_out, out_stride);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_err(err, std::string("mlxf: kernel launch failed: ") + hipGetErrorString(e));
    return MLXF_EHIP;
  }
  return MLXF_OK;
}
