/*
 * mlxf_sampler.h -- C ABI of the MI355X (gfx950) batched token sampler.
 *
 * Drop-in for the decode step's sampler boundary of hvasconcelos/mlxforge:
 *   Sampler::sample(logits, params, key[, history])  src/sample/sampler.h:51-58
 *   Sampler::greedy(logits)                           src/sample/sampler.h:61
 * as driven row by row by Worker::sample_rows / finalize_sample
 * (src/runtime/worker.cpp:448-514).  One call samples every row of a [B, V]
 * logits matrix with per-row parameters, asynchronously on the caller's HIP
 * stream (the analogue of the reference's single mx::async_eval per step,
 * src/runtime/worker.cpp:498).
 *
 * Conventions (mirroring the reference's product C ABI, src/capi/mlxforge.h:10-23):
 *   - no C++ types cross this boundary; every pointer named d_* is device memory;
 *   - every fallible call returns 0 on success or a negative MLXF_E* code, and if
 *     `err` is non-NULL sets *err to a malloc'd message the caller releases with
 *     mlxf_string_free();
 *   - no exception ever crosses the boundary;
 *   - the library allocates nothing in mlxf_sample / mlxf_greedy: scratch is the
 *     caller-provided workspace (size from mlxf_sampler_workspace_size); it
 *     needs no initialisation (each call clears what it counts in);
 *   - calls are reentrant per stream; two calls that share a workspace must be
 *     ordered on one stream.
 */
#ifndef MLXF_SAMPLER_H
#define MLXF_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MLXF_SAMPLER_ABI_VERSION 1

/* Logits element types.  Production logits are fp16 (src/model/decoder_model.cpp:368). */
#define MLXF_DTYPE_F32 0
#define MLXF_DTYPE_BF16 1
#define MLXF_DTYPE_F16 2

/* Return codes. */
#define MLXF_OK 0
#define MLXF_EINVAL (-1)     /* bad argument (shape, dtype, NULL pointer, alignment) */
#define MLXF_EWORKSPACE (-2) /* workspace NULL or smaller than mlxf_sampler_workspace_size */
#define MLXF_EHIP (-3)       /* a HIP runtime call or kernel launch failed */

/* Largest top_logprobs column count supported per call.  The reference's HTTP
 * layer admits top_logprobs in [0, 20] (src/server/openai.cpp:150-152), its
 * sampler any K = min(top_logprobs, V) (src/sample/sampler.cpp:52).  Up to 64
 * columns come out of the sampling kernels' best-64 lists; a call with K_max
 * above 64 adds one kernel that selects and sorts every row's K (one
 * workgroup per row, K sorted in LDS). */
#define MLXF_MAX_TOP_LOGPROBS 4096
/* Largest vocabulary accepted: at most 64 slices of 8192 logits per row. */
#define MLXF_MAX_VOCAB 524288

/* ABI version of the loaded library (MLXF_SAMPLER_ABI_VERSION it was built with).
 * No reference counterpart for the sampler itself; mirrors mlxforge_abi_version
 * (src/capi/mlxforge.h:56). */
int mlxf_sampler_abi_version(void);

/* Bytes of device workspace mlxf_sample / mlxf_greedy need for this shape.
 * Replaces the lazily allocated MLX temporaries of Sampler::sample
 * (src/sample/sampler.cpp:141-166); the caller owns and reuses the buffer. */
int mlxf_sampler_workspace_size(int B, int V, int K_max, int dtype, size_t* bytes, char** err);

/* Zero the per-row counters at the start of a workspace with a fill kernel on
 * `stream` (no hipMemset, so it may be captured in a graph).  Kept for
 * callers of ABI version 1; no call needs it any more (each call clears its
 * counters itself).  No reference counterpart. */
int mlxf_sampler_workspace_init(void* d_workspace, size_t workspace_bytes, void* stream,
                                char** err);

/* Sample one token per row.  Replaces the per-row loop of Worker::sample_rows
 * (src/runtime/worker.cpp:453-483) calling Sampler::sample
 * (src/sample/sampler.cpp:141-166), with the MLX random::categorical draw
 * (src/sample/sampler.cpp:165) replaced by an inverse-CDF draw from a
 * caller-supplied uniform per row.
 *
 *   d_logits        [B, row_stride] elements of `dtype`; row r is
 *                   d_logits + r * row_stride, only its first V entries are read
 *                   (row_stride > V covers the bucket-padded (bucket, 1, V) view,
 *                   src/runtime/worker.cpp:533).
 *   d_temperature   [B] fp32 or NULL (NULL: every row greedy).  A row is greedy
 *                   when T <= 0 or T is not finite (src/sample/sampler.h:16,
 *                   src/capi/mlxforge.cpp:55).  T is rounded to `dtype` before
 *                   dividing (src/sample/sampler.cpp:158).
 *   d_top_k         [B] int32 or NULL.  <= 0 disables; clamped to V
 *                   (src/sample/sampler.cpp:159-161).  Ties at the k-th value are kept.
 *   d_top_p         [B] fp32 or NULL.  Active when 0 < p < 1, else disabled
 *                   (src/capi/mlxforge.cpp:57); applied after top-k.
 *   d_top_logprobs  [B] int32 or NULL (NULL: all -1).  -1: no logprob work for the
 *                   row (out_logprobs[r] = NaN); 0: chosen-token logprob only;
 *                   N > 0: also the min(N, K_max, V) most likely alternatives
 *                   (src/sample/sampler.h:24-29, src/runtime/worker.cpp:477).
 *   d_uniforms      [B] fp32 in [0, 1), one per row; may be NULL only when
 *                   d_temperature is NULL.  Values outside [0, 1) are clamped.
 *   d_out_ids       [B] int32 sampled token ids.
 *   d_out_logprobs  [B] fp32 or NULL: log_softmax of the unscaled logits at the
 *                   chosen id (src/sample/sampler.cpp:146-154).
 *   d_out_top_ids, d_out_top_logprobs
 *                   [B, K_max] (NULL allowed when K_max == 0): alternatives in
 *                   descending logprob order, ties by ascending id; unused
 *                   columns hold id -1 and logprob -inf.
 *   d_workspace     >= mlxf_sampler_workspace_size(B, V, K_max, dtype) bytes,
 *                   256-byte aligned.
 *   stream          hipStream_t (NULL = the default stream).
 */
int mlxf_sample(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                const int32_t* d_top_logprobs, const float* d_uniforms, int32_t* d_out_ids,
                float* d_out_logprobs, int32_t* d_out_top_ids, float* d_out_top_logprobs,
                int K_max, void* d_workspace, size_t workspace_bytes, void* stream, char** err);

/* mlxf_sample with the number of refine stages to launch (0..3) given by the
 * caller.  mlxf_sample launches two, the most mlxf_sampler_refine_stages ever
 * asks for (a third measured slower on every configuration: the rows it would
 * serve finish sooner in the second stage's deciding kernel); a caller that
 * knows its rows' parameters on the host (as Worker::sample_rows does,
 * src/runtime/worker.cpp:453-473) passes mlxf_sampler_refine_stages(...)
 * instead and skips launches no row can use.  Results are identical for every
 * count: rows still open after the last stage launched are finished by its
 * deciding kernel.  No reference counterpart (the reference builds one MLX
 * graph per row). */
int mlxf_sample_staged(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                       const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                       const int32_t* d_top_logprobs, const float* d_uniforms, int32_t* d_out_ids,
                       float* d_out_logprobs, int32_t* d_out_top_ids, float* d_out_top_logprobs,
                       int K_max, void* d_workspace, size_t workspace_bytes, int refine_stages,
                       void* stream, char** err);

/* mlxf_sample_staged with per-row min_p as well (src/sample/sampler.h:19,
 * applied after top-p as in src/sample/sampler.cpp:163 and :87-93):
 *   d_min_p   [B] fp32 or NULL (NULL: every row off).  Active when
 *             0 < min_p <= 1, else off (src/capi/mlxforge.cpp:58); rounded to
 *             the logits dtype; keeps the tokens whose exp(z' - max z')
 *             reaches it.
 * The stage hint of mlxf_sampler_refine_stages holds unchanged (a row whose
 * min_p cuts deeper than its top-k / top-p takes one more pass, which the last
 * launched stage runs itself when no stage is left). */
int mlxf_sample_ex(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                   const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                   const float* d_min_p, const int32_t* d_top_logprobs, const float* d_uniforms,
                   int32_t* d_out_ids, float* d_out_logprobs, int32_t* d_out_top_ids,
                   float* d_out_top_logprobs, int K_max, void* d_workspace, size_t workspace_bytes,
                   int refine_stages, void* stream, char** err);

/* Bytes of the fixed scratch mlxf_sample_noalloc holds on each GPU it runs on
 * (from that GPU's first call until the process ends). */
#define MLXF_NOALLOC_SCRATCH_BYTES (64u << 20)

/* mlxf_sample_ex without a workspace argument: the call allocates nothing and
 * takes no caller memory besides its inputs and outputs, for callers that
 * cannot allocate device memory or hold a workspace (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  No
 * counterpart in the reference (its MLX temporaries are allocated per call).
 *
 * Scratch is a fixed MLXF_NOALLOC_SCRATCH_BYTES array in device memory, one
 * per GPU, shared by every call on that GPU and kept between calls: calls that
 * may overlap on one GPU (on different streams, or from different threads)
 * race and must be ordered by the caller.  Its device address is looked up on
 * the stream's GPU at that GPU's first call.  Shapes whose workspace
 * (mlxf_sampler_workspace_size) exceeds the scratch are refused with
 * MLXF_EWORKSPACE; B = 256 rows of V = 262144 fit.  Arguments and results are
 * those of mlxf_sample_ex. */
int mlxf_sample_noalloc(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                        const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                        const float* d_min_p, const int32_t* d_top_logprobs, const float* d_uniforms,
                        int32_t* d_out_ids, float* d_out_logprobs, int32_t* d_out_top_ids,
                        float* d_out_top_logprobs, int K_max, int refine_stages, void* stream,
                        char** err);

/* Refine stages a call needs, from HOST copies of the per-row temperature,
 * top_k and top_p (NULL = the sentinel: greedy / off / off), with the same
 * sanitisation as mlxf_sample (src/sample/sampler.h:16-29,
 * src/capi/mlxforge.cpp:43-70): 0 when every row is greedy or has a top-k of
 * at most 63, 1 when every other row is temperature-only, else 2 (a row still
 * open after the second stage is finished by its deciding kernel, which
 * measured faster than a third stage). */
int mlxf_sampler_refine_stages(int B, int V, int dtype, const float* h_temperature,
                               const int32_t* h_top_k, const float* h_top_p);

/* The first kernel of mlxf_sample alone -- the one HBM read of the logits
 * (per-slice maxima, log-sum-exp partials, best-64 lists), which dominates a
 * decode step -- with the same arguments; writes no output.  For measuring
 * that kernel in isolation.  No reference counterpart. */
int mlxf_sampler_first_pass(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                            const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                            const int32_t* d_top_logprobs, const float* d_uniforms, int32_t* d_out_ids,
                            float* d_out_logprobs, int32_t* d_out_top_ids, float* d_out_top_logprobs,
                            int K_max, void* d_workspace, size_t workspace_bytes, void* stream, char** err);

/* Bytes of device workspace mlxf_apply_penalties needs: one 32-bit counter per
 * (row, vocabulary id).  Zero it once before first use; every call leaves it
 * zero.  No reference counterpart (MLX allocates the counts per call). */
int mlxf_penalties_workspace_size(int B, int V, size_t* bytes, char** err);

/* Repetition / frequency / presence penalties applied to the logits IN PLACE,
 * before mlxf_sample / mlxf_greedy on the same logits: the penalized `adj` of
 * Sampler::sample (src/sample/sampler.cpp:122-133, used at :144; the worker
 * passes the history only to rows with penalties, src/runtime/worker.cpp:469).
 * Only the logits at history ids change:
 *   repetition  z > 0 ? z / pen : z * pen         (sampler.cpp:95-105)
 *   then        z - count * frequency - presence  (sampler.cpp:107-120)
 * each step rounded to the logits dtype, with pen, frequency, presence and the
 * id's count in the history as values of that dtype.  NaN logits are left
 * as they are.
 *   d_logits      [B, row_stride] of `dtype`, modified in place.
 *   d_history     [B, hist_stride] int32 token ids; row r uses its first
 *                 d_hist_len[r] entries (d_hist_len NULL: all hist_stride).
 *                 Ids outside [0, V) are ignored.
 *   d_repetition  [B] fp32 or NULL (1 = off; not finite and positive: off).
 *   d_frequency, d_presence
 *                 [B] fp32 or NULL (0 = off; not finite: off)
 *                 (src/capi/mlxforge.cpp:59-64).
 *   d_workspace   >= mlxf_penalties_workspace_size(B, V) bytes, zeroed once.
 * Two kernels on `stream`; no allocation. */
int mlxf_apply_penalties(void* d_logits, int dtype, int B, int V, int64_t row_stride,
                         const int32_t* d_history, int64_t hist_stride, const int32_t* d_hist_len,
                         const float* d_repetition, const float* d_frequency, const float* d_presence,
                         void* d_workspace, size_t workspace_bytes, void* stream, char** err);

/* Per-row draw uniforms on the device: u[r] = Philox4x32-10 keyed by
 * d_seed[r] at counter (step_r, 0), first word's top 24 bits times 2^-24, in
 * [0, 1).  step_r = d_step[r], or `step` when d_step is NULL.  Replaces the
 * per-row MLX key derived from the request seed and split every step
 * (src/runtime/worker.cpp:416,465-466): the same (seed, step) gives the same
 * uniform, so a seed replays its tokens (tests/sample/sampler_test.cpp:126-134).
 * One small kernel on `stream`; feed d_uniforms to mlxf_sample*. */
int mlxf_uniforms(int B, const uint64_t* d_seed, const uint64_t* d_step, uint64_t step,
                  float* d_uniforms, void* stream, char** err);

/* The grammar-constrained rows of a step: row + an additive fp32 mask of
 * 0 / -inf, which MLX evaluates as an fp32 row (src/runtime/worker.cpp:455-459;
 * the mask, :142-179).  The mask is given as one bit per token, 1 = allowed:
 *   d_allowed_bits  [B, bits_stride] uint32 words, bit (i & 31) of word i >> 5.
 * Writes d_out [B, out_stride] fp32: the logit where allowed, -inf elsewhere.
 * A row with no allowed token is copied unmasked (the reference never builds
 * an all -inf mask, :175-177).  Sample d_out with dtype MLXF_DTYPE_F32, as the
 * reference samples the promoted row.  No reference counterpart for the bit
 * packing (the reference uploads the fp32 array). */
int mlxf_apply_mask(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                    const uint32_t* d_allowed_bits, int64_t bits_stride, float* d_out,
                    int64_t out_stride, void* stream, char** err);

/* The reference's filter helpers (src/sample/sampler.h:63-69; graph ops that
 * return the logits with every removed entry set to -inf), on a [B, V] matrix:
 *   mlxf_apply_top_k  Sampler::apply_top_k (src/sample/sampler.cpp:63-68): keep
 *                     the entries at or above the k-th largest, counting
 *                     multiplicity (ties there are kept, so more than k can
 *                     remain); k clamped to V (:159-161); k <= 0 keeps all.
 *   mlxf_apply_top_p  Sampler::apply_top_p (:70-85): keep the smallest prefix
 *                     in (value desc, index asc) order whose prior mass is
 *                     below p; p outside (0, 1) keeps all.
 *   mlxf_apply_min_p  Sampler::apply_min_p (:87-93): keep the entries whose
 *                     probability reaches min_p times the largest; min_p
 *                     outside (0, 1] keeps all.
 *   mlxf_filter_logits  all three after the temperature division, per row,
 *                     as Sampler::sample applies them (:158-163): writes z' =
 *                     round_dtype(z / T) (T <= 0, non-finite or NULL: no
 *                     division) with the removed entries at -inf.  NULL
 *                     arrays: that filter off.
 * The kept sets are the sampling call's, with its masses and tie rules
 * (top-p order is value desc, index asc; the mass is summed in fixed point,
 * so it does not depend on the summation order); NaN logits read as -inf.
 * d_out has the logits' dtype; it may be d_logits itself (in place,
 * out_stride == row_stride) but must not overlap it otherwise.
 *   d_workspace   >= mlxf_filter_workspace_size(B, V) bytes, 256-byte aligned;
 *                 no initialisation needed (every call writes what it reads).
 * Up to ten kernels on `stream` (fewer for the single-filter calls), each over
 * every row with several workgroups per row; no allocation.  A helper, not
 * the decode step's path. */
int mlxf_filter_workspace_size(int B, int V, size_t* bytes, char** err);
int mlxf_filter_logits(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                       const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                       const float* d_min_p, void* d_out, int64_t out_stride, void* d_workspace,
                       size_t workspace_bytes, void* stream, char** err);
int mlxf_apply_top_k(const void* d_logits, int dtype, int B, int V, int64_t row_stride, int k,
                     void* d_out, int64_t out_stride, void* d_workspace, size_t workspace_bytes,
                     void* stream, char** err);
int mlxf_apply_top_p(const void* d_logits, int dtype, int B, int V, int64_t row_stride, float p,
                     void* d_out, int64_t out_stride, void* d_workspace, size_t workspace_bytes,
                     void* stream, char** err);
int mlxf_apply_min_p(const void* d_logits, int dtype, int B, int V, int64_t row_stride, float min_p,
                     void* d_out, int64_t out_stride, void* d_workspace, size_t workspace_bytes,
                     void* stream, char** err);

/* argmax over each row, lowest index on ties: Sampler::greedy
 * (src/sample/sampler.h:61, src/sample/sampler.cpp:59-61). */
int mlxf_greedy(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                int32_t* d_out_ids, void* d_workspace, size_t workspace_bytes, void* stream,
                char** err);

/* Release a message returned through `err` (mirrors mlxforge_string_free). */
void mlxf_string_free(char* s);

#ifdef __cplusplus
}
#endif

#endif /* MLXF_SAMPLER_H */
