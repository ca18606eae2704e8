// sampler_f16.hip -- the sampler kernels for f16 logits.
#include "sampler_impl.hpp"

namespace mlxf {

hipError_t launch_f16(const Args& a, int ept, bool vecok, int nst, hipStream_t st) {
  return launch_dt<MLXF_DTYPE_F16>(a, ept, vecok, nst, st);
}

}  // namespace mlxf
