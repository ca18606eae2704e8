// uniforms.hip -- per-row draw uniforms on the device, replacing the MLX key
// the reference derives from the request seed and splits every decode step
// (random::key / split, src/runtime/worker.cpp:416,465-466; reproducibility
// per seed, tests/sample/sampler_test.cpp:126-134).
//
// Counter-based: u = Philox4x32-10 (J. Salmon, M. Moraes, R. Dror, D. Shaw,
// "Parallel random numbers: as easy as 1, 2, 3", SC'11) keyed by the row's
// 64-bit seed, at counter (step, 0) -- so a row's uniform is a pure function
// of (seed, step): the same seed replays the same tokens, and steps draw
// independently.  The first output word's top 24 bits give u = x * 2^-24 in
// [0, 1 - 2^-24].
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <string>

#include "mlxf_sampler.h"

namespace mlxf {
namespace {

__device__ __forceinline__ unsigned int philox_u32(unsigned long long seed, unsigned long long step) {
  unsigned int c0 = static_cast<unsigned int>(step), c1 = static_cast<unsigned int>(step >> 32);
  unsigned int c2 = 0u, c3 = 0u;
  unsigned int k0 = static_cast<unsigned int>(seed), k1 = static_cast<unsigned int>(seed >> 32);
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const unsigned int lo0 = 0xD2511F53u * c0, hi0 = __umulhi(0xD2511F53u, c0);
    const unsigned int lo1 = 0xCD9E8D57u * c2, hi1 = __umulhi(0xCD9E8D57u, c2);
    const unsigned int n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0;
    c1 = lo1;
    c2 = n2;
    c3 = lo0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  return c0;
}

__global__ __launch_bounds__(256) void k_uniforms(int B, const unsigned long long* seed,
                                                  const unsigned long long* step, unsigned long long step0,
                                                  float* u) {
  const int r = static_cast<int>(blockIdx.x) * 256 + static_cast<int>(threadIdx.x);
  if (r >= B) return;
  const unsigned int x = philox_u32(seed[r], step ? step[r] : step0);
  u[r] = static_cast<float>(x >> 8) * 0x1p-24f;
}

void set_err(char** err, const std::string& msg) {
  if (!err) return;
  char* q = static_cast<char*>(std::malloc(msg.size() + 1));
  if (q) std::memcpy(q, msg.c_str(), msg.size() + 1);
  *err = q;
}

}  // namespace
}  // namespace mlxf

extern "C" int mlxf_uniforms(int B, const uint64_t* d_seed, const uint64_t* d_step, uint64_t step,
                             float* d_uniforms, void* stream, char** err) {
  if (B < 0) {
    mlxf::set_err(err, "mlxf: B must be >= 0");
    return MLXF_EINVAL;
  }
  if (B == 0) return MLXF_OK;
  if (!d_seed || !d_uniforms) {
    mlxf::set_err(err, "mlxf: d_seed and d_uniforms must not be NULL");
    return MLXF_EINVAL;
  }
  hipLaunchKernelGGL(mlxf::k_uniforms, dim3(static_cast<unsigned int>((B + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), B,
                     reinterpret_cast<const unsigned long long*>(d_seed),
                     reinterpret_cast<const unsigned long long*>(d_step),
                     static_cast<unsigned long long>(step), d_uniforms);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    mlxf::set_err(err, std::string("mlxf: kernel launch failed: ") + hipGetErrorString(e));
    return MLXF_EHIP;
  }
  return MLXF_OK;
}
