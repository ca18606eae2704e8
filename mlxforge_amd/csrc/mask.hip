// mask.hip -- the grammar-constrained row of the decode step: logits plus an
// additive fp32 mask of 0 (allowed) / -inf (disallowed), which MLX evaluates
// as an fp32 row (src/runtime/worker.cpp:455-459, the mask built at :142-179).
// Here the mask arrives as one bit per token (1 = allowed), 1/32 of the fp32
// array, and the kernel writes the fp32 row: the logit where allowed, -inf
// elsewhere -- the exact value of row + mask.  A row with no allowed token is
// copied unmasked: the reference never builds an all -inf mask and adds zeros
// instead (:175-177).  The masked rows are then sampled as fp32 logits.
//
// One workgroup per slice of MASK_SLICE tokens (8 per thread: one or two
// 16-byte loads, two 16-byte stores, one byte of the bit mask), so a row is
// spread over many CUs.  A slice with an allowed token knows the row has one;
// a slice without scans the row's whole bit mask (16-byte loads; it is in L2
// after the first such slice) to tell an all-disallowed row.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <string>

#include "device_common.hpp"
#include "mlxf_sampler.h"

namespace mlxf {
namespace {

constexpr int MASK_THREADS = 256;
constexpr int MASK_EPT = 8;
constexpr int MASK_SLICE = MASK_THREADS * MASK_EPT;

// Any allowed token among the row's nw bit words (bits past V do not count)?
// Whole workgroup; `flag` is one LDS word.
__device__ __forceinline__ bool row_any_allowed(const unsigned int* b, int V, int* flag) {
  const int tid = static_cast<int>(threadIdx.x);
  const int nw = (V + 31) / 32;
  const unsigned int last = (V & 31) ? (1u << (V & 31)) - 1u : 0xffffffffu;
  unsigned int acc = 0u;
  const bool vec = (reinterpret_cast<uintptr_t>(b) & 15u) == 0;
  if (vec) {
    const uint4* b4 = reinterpret_cast<const uint4*>(b);
    for (int q = tid; q < nw / 4; q += MASK_THREADS) {
      const uint4 x = b4[q];
      const int w = 4 * q;
      acc |= x.x & (w == nw - 1 ? last : ~0u);
      acc |= x.y & (w + 1 == nw - 1 ? last : ~0u);
      acc |= x.z & (w + 2 == nw - 1 ? last : ~0u);
      acc |= x.w & (w + 3 == nw - 1 ? last : ~0u);
    }
    for (int w = (nw / 4) * 4 + tid; w < nw; w += MASK_THREADS) acc |= b[w] & (w == nw - 1 ? last : ~0u);
  } else {
    for (int w = tid; w < nw; w += MASK_THREADS) acc |= b[w] & (w == nw - 1 ? last : ~0u);
  }
  if (tid == 0) *flag = 0;
  __syncthreads();
  if (__builtin_amdgcn_ballot_w64(acc != 0u) && (tid & 63) == 0) *flag = 1;
  __syncthreads();
  return *flag != 0;
}

template <int DT, bool VECIN, bool VECOUT>
__global__ __launch_bounds__(MASK_THREADS) void k_mask(const void* logits, long long row_stride, int V,
                                                       const unsigned int* bits, long long bits_stride,
                                                       float* out, long long out_stride) {
  __shared__ int flag[2];
  const int r = static_cast<int>(blockIdx.y);
  const int tid = static_cast<int>(threadIdx.x);
  const int i0 = static_cast<int>(blockIdx.x) * MASK_SLICE + tid * MASK_EPT;
  const unsigned int* b = bits + static_cast<size_t>(r) * static_cast<size_t>(bits_stride);
  const char* row = static_cast<const char*>(logits) + static_cast<size_t>(r) * static_cast<size_t>(row_stride) * elem_size<DT>();
  float* o = out + static_cast<size_t>(r) * static_cast<size_t>(out_stride);
  const int n = min(MASK_EPT, V - i0);  // this thread's tokens (may be <= 0 in the last slice)
  float z[MASK_EPT];
  if (n == MASK_EPT && VECIN) {
    if constexpr (DT == MLXF_DTYPE_F32) {
      const float4* p = reinterpret_cast<const float4*>(row + static_cast<size_t>(i0) * 4);
      const float4 a = p[0], c = p[1];
      z[0] = a.x; z[1] = a.y; z[2] = a.z; z[3] = a.w;
      z[4] = c.x; z[5] = c.y; z[6] = c.z; z[7] = c.w;
    } else {
      const uint4 q = *reinterpret_cast<const uint4*>(row + static_cast<size_t>(i0) * 2);
      const unsigned int w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (DT == MLXF_DTYPE_BF16) {
          z[2 * j] = __uint_as_float(w[j] << 16);
          z[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        } else {
          __half_raw lo, hi;
          lo.x = static_cast<unsigned short>(w[j] & 0xffffu);
          hi.x = static_cast<unsigned short>(w[j] >> 16);
          z[2 * j] = __half2float(__half(lo));
          z[2 * j + 1] = __half2float(__half(hi));
        }
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < MASK_EPT; ++j) {
      float v = 0.0f;
      if (j < n) {
        if constexpr (DT == MLXF_DTYPE_F32)
          v = reinterpret_cast<const float*>(row)[i0 + j];
        else if constexpr (DT == MLXF_DTYPE_BF16)
          v = __uint_as_float(static_cast<unsigned int>(reinterpret_cast<const unsigned short*>(row)[i0 + j]) << 16);
        else
          v = __half2float(reinterpret_cast<const __half*>(row)[i0 + j]);
      }
      z[j] = v;
    }
  }
  // this thread's 8 mask bits (i0 is a multiple of 8), none past V
  unsigned int m = n > 0 ? (b[i0 >> 5] >> (i0 & 31)) & 0xffu : 0u;
  if (n < MASK_EPT) m &= n > 0 ? (1u << n) - 1u : 0u;
  // a slice with an allowed token: the row has one; else look at the whole row
  if (tid == 0) flag[1] = 0;
  __syncthreads();
  if (__builtin_amdgcn_ballot_w64(m != 0u) && (tid & 63) == 0) flag[1] = 1;
  __syncthreads();
  const bool any = flag[1] != 0 || row_any_allowed(b, V, &flag[0]);
  if (!any) m = 0xffu;  // no allowed token in the row: copied unmasked
  float y[MASK_EPT];
#pragma unroll
  for (int j = 0; j < MASK_EPT; ++j) y[j] = ((m >> j) & 1u) ? z[j] : -INFINITY;
  if (n == MASK_EPT && VECOUT) {
    float4* q = reinterpret_cast<float4*>(o + i0);
    q[0] = make_float4(y[0], y[1], y[2], y[3]);
    q[1] = make_float4(y[4], y[5], y[6], y[7]);
  } else {
#pragma unroll
    for (int j = 0; j < MASK_EPT; ++j)
      if (j < n) o[i0 + j] = y[j];
  }
}

template <int DT>
void launch_mask(dim3 grid, hipStream_t st, bool vin, bool vout, const void* logits, long long row_stride, int V,
                 const unsigned int* bits, long long bits_stride, float* out, long long out_stride) {
  if (vin && vout)
    hipLaunchKernelGGL((k_mask<DT, true, true>), grid, dim3(MASK_THREADS), 0, st, logits, row_stride, V, bits,
                       bits_stride, out, out_stride);
  else if (vin)
    hipLaunchKernelGGL((k_mask<DT, true, false>), grid, dim3(MASK_THREADS), 0, st, logits, row_stride, V, bits,
                       bits_stride, out, out_stride);
  else if (vout)
    hipLaunchKernelGGL((k_mask<DT, false, true>), grid, dim3(MASK_THREADS), 0, st, logits, row_stride, V, bits,
                       bits_stride, out, out_stride);
  else
    hipLaunchKernelGGL((k_mask<DT, false, false>), grid, dim3(MASK_THREADS), 0, st, logits, row_stride, V, bits,
                       bits_stride, out, out_stride);
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
  if (B < 0 || B > 65535 || V < 1 || V > MLXF_MAX_VOCAB || row_stride < V || out_stride < V ||
      bits_stride < (V + 31) / 32) {
    set_err(err, "mlxf: bad shape (B in [0, 65535], V in [1, MLXF_MAX_VOCAB], row_stride and out_stride >= V, "
                 "bits_stride >= ceil(V / 32))");
    return MLXF_EINVAL;
  }
  if (B == 0) return MLXF_OK;
  if (!d_logits || !d_allowed_bits || !d_out) {
    set_err(err, "mlxf: d_logits, d_allowed_bits and d_out must not be NULL");
    return MLXF_EINVAL;
  }
  const size_t esz = dtype == MLXF_DTYPE_F32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(d_logits) % esz) || (reinterpret_cast<uintptr_t>(d_out) % 4) ||
      (reinterpret_cast<uintptr_t>(d_allowed_bits) % 4)) {
    set_err(err, "mlxf: d_logits, d_allowed_bits or d_out is not aligned to its element size");
    return MLXF_EINVAL;
  }
  // 16-byte loads and stores when every row start is 16-byte aligned
  const bool vin = reinterpret_cast<uintptr_t>(d_logits) % 16 == 0 && (static_cast<size_t>(row_stride) * esz) % 16 == 0;
  const bool vout = reinterpret_cast<uintptr_t>(d_out) % 16 == 0 && (static_cast<size_t>(out_stride) * 4) % 16 == 0;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned int>((V + MASK_SLICE - 1) / MASK_SLICE), static_cast<unsigned int>(B));
  const unsigned int* bits = reinterpret_cast<const unsigned int*>(d_allowed_bits);
  if (dtype == MLXF_DTYPE_F32)
    launch_mask<MLXF_DTYPE_F32>(grid, st, vin, vout, d_logits, row_stride, V, bits, bits_stride, d_out, out_stride);
  else if (dtype == MLXF_DTYPE_BF16)
    launch_mask<MLXF_DTYPE_BF16>(grid, st, vin, vout, d_logits, row_stride, V, bits, bits_stride, d_out, out_stride);
  else
    launch_mask<MLXF_DTYPE_F16>(grid, st, vin, vout, d_logits, row_stride, V, bits, bits_stride, d_out, out_stride);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_err(err, std::string("mlxf: kernel launch failed: ") + hipGetErrorString(e));
    return MLXF_EHIP;
  }
  return MLXF_OK;
}
