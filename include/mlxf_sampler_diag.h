/*
 * mlxf_sampler_diag.h -- diagnostic entry point of libmlxf_sampler.so.
 *
 * Not part of the drop-in boundary (no reference counterpart): a twin of
 * mlxf_sample used by the benchmark to time each stage of the launch sequence
 * with HIP events on the caller's stream.
 */
#ifndef MLXF_SAMPLER_DIAG_H
#define MLXF_SAMPLER_DIAG_H

#include "mlxf_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Number of kernels in one mlxf_sample launch sequence and their order:
 * 0 scan, 1 plan, 2 extract, 3 select, 4 draw. */
#define MLXF_NUM_STAGES 5

/* Same arguments and results as mlxf_sample, plus stage_ms[MLXF_NUM_STAGES]
 * (host memory): the elapsed time of each kernel, measured with a HIP event
 * recorded before and after it on `stream`.  Synchronizes the stream; creates
 * and destroys its events on every call. */
int mlxf_sample_profiled(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                         const float* d_temperature, const int32_t* d_top_k,
                         const float* d_top_p, const int32_t* d_top_logprobs,
                         const float* d_uniforms, int32_t* d_out_ids, float* d_out_logprobs,
                         int32_t* d_out_top_ids, float* d_out_top_logprobs, int K_max,
                         void* d_workspace, size_t workspace_bytes, void* stream,
                         float* stage_ms, char** err);

#ifdef __cplusplus
}
#endif

#endif /* MLXF_SAMPLER_DIAG_H */
