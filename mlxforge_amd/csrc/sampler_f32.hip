// sampler_f32.hip -- the sampler kernels for f32 logits.
#include "sampler_impl.hpp"

namespace mlxf {

hipError_t launch_f32(const Args& a, int ept, bool vecok, int nst, hipStream_t st) {
  return launch_dt<MLXF_DTYPE_F32>(a, ept, vecok, nst, st);
}

}  // namespace mlxf
