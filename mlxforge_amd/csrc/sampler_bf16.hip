// sampler_bf16.hip -- the sampler kernels for bf16 logits.
#include "sampler_impl.hpp"

namespace mlxf {

hipError_t launch_bf16(const Args& a, int ept, bool vecok, int nst, hipStream_t st) {
  return launch_dt<MLXF_DTYPE_BF16>(a, ept, vecok, nst, st);
}

hipError_t launch_row16_bf16(const Args& a, int ept, const RhArgs& x, hipStream_t st) {
  return launch_row16_dt<MLXF_DTYPE_BF16>(a, ept, x, st);
}

}  // namespace mlxf
