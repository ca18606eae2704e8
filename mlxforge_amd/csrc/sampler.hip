// sampler.hip -- host side of the MI355X (gfx950) batched token sampler
// behind the C ABI in include/mlxf_sampler.h: workspace layout, argument
// checks, the stage count, and the launch of one dtype's kernel sequence
// (sampler_impl.hpp, instantiated per dtype in sampler_<dtype>.hip).
#include <mutex>

#include "sampler_impl.hpp"

// Scratch of the allocation-free entry point, mlxf_sample_noalloc: one copy per
// GPU, held from the library's first use on that GPU until the process ends.
// In host code `scratch` only names the symbol; the device address of each
// GPU's copy comes from hipGetSymbolAddress (noalloc_scratch below).
static __device__ __align__(256) unsigned char scratch[MLXF_NOALLOC_SCRATCH_BYTES];

namespace mlxf {
namespace {

// Zero the per-row counters of a fresh workspace.
__global__ void k_zero(unsigned int* p, size_t n) {
  const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

struct Layout {
  int S, L, EPT;
  size_t off_ncand, off_actcnt, off_actlist, off_rec, off_list, off_rowst, off_hcnt, off_hmass, off_above,
      off_dsum, off_cand, off_hsplit, off_crec, off_wide, total;
};

// bf16 rows with no top_logprobs take the row-histogram path (rowhist.hpp):
// one workgroup per row counts the row into exact per-value histograms and
// decides everything from them.  It serves every stage count alike (it has
// no refine stages), but not the first-pass-only timing call (nst < 0).  With
// at most ROW_SPLIT_MAX_B rows (four chunk workgroups per row still fit the
// 256 CUs at once) the chunks are counted by their own workgroups first.
// With more rows each workgroup counts its row with 16-bit counters for the
// two halves of each chunk, so no half may hold more than 65535 logits: an
// even number of iterations per chunk, at most 7 per half (V <= 458752; larger
// vocabularies with that many rows take the per-slice path).
constexpr int ROW_ITER_LOGITS = 1024 * 8;              // logits per pass-1 iteration
constexpr int ROW_CHUNK_LOGITS = 4 * ROW_ITER_LOGITS;  // logits per chunk iteration count
constexpr int ROW_MIN_V = 32768;
constexpr int ROW_SPLIT_MAX_B = 64;
constexpr int ROW_PACK_MAX_V = 4 * 2 * 7 * ROW_ITER_LOGITS;
bool row_split(int dtype, int B, int V) { return dtype == MLXF_DTYPE_BF16 && V >= ROW_MIN_V && B <= ROW_SPLIT_MAX_B; }
bool use_row_path(int dtype, int B, int V, int K_max, bool vecok, int nst) {
  return dtype == MLXF_DTYPE_BF16 && K_max == 0 && vecok && nst >= 0 && V >= ROW_MIN_V &&
         (row_split(dtype, B, V) || V <= ROW_PACK_MAX_V);
}

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// The head of the workspace, at offsets that do not depend on the shape: per-row
// gathered-candidate counters (65536 32-bit words) and the stage-list counts.
// The first kernel of every call clears the stage-list counts and the counters
// of its rows, so a workspace needs no initialisation and a call never depends
// on what an earlier (possibly failed) call left behind.
constexpr size_t ROWS_MAX = 65536;
constexpr size_t CTR_BYTES_MAX = ROWS_MAX * sizeof(unsigned int) + 256;

// EPT: the largest of {32, 16, 8} that still gives at least one workgroup per
// CU (256) with at most MAX_S slices per row; otherwise the smallest EPT with
// S <= MAX_S.
Layout make_layout(int B, int V, int K_max, int dtype) {
  Layout l;
  int ept = 0;
  for (int e : {32, 16, 8}) {
    const int L = THREADS * e;
    const int S = (V + L - 1) / L;
    if (S <= MAX_S && static_cast<long long>(B) * S >= 256) {
      ept = e;
      break;
    }
  }
  if (!ept) {
    for (int e : {8, 16, 32}) {
      const int L = THREADS * e;
      if ((V + L - 1) / L <= MAX_S) {
        ept = e;
        break;
      }
    }
  }
  l.EPT = ept;
  l.L = THREADS * ept;
  l.S = (V + l.L - 1) / l.L;
  const size_t BS = static_cast<size_t>(B) * l.S;
  const size_t nb = B > 0 ? static_cast<size_t>(B) : 1;
  l.off_ncand = 0;
  l.off_actcnt = ROWS_MAX * sizeof(unsigned int);
  size_t o = align256(CTR_BYTES_MAX);
  l.off_actlist = o;
  o = align256(o + sizeof(unsigned int) * NSTAGE * nb);
  l.off_rec = o;
  o = align256(o + REC * sizeof(unsigned long long) * BS);
  l.off_list = o;
  o = align256(o + sizeof(unsigned long long) * BS * SCAP);
  l.off_rowst = o;
  o = align256(o + sizeof(unsigned long long) * RS_WORDS * nb);
  l.off_hcnt = o;
  o = align256(o + sizeof(unsigned int) * BS * NB);
  l.off_hmass = o;
  o = align256(o + sizeof(unsigned long long) * BS * NB);
  l.off_above = o;
  o = align256(o + sizeof(unsigned long long) * BS);
  l.off_dsum = o;
  o = align256(o + sizeof(unsigned long long) * BS);
  l.off_cand = o;
  o = align256(o + sizeof(unsigned long long) * nb * CAP);
  // the row-histogram path's split chunk histograms and chunk records
  const size_t nsplit = row_split(dtype, B, V) ? nb : 0;
  l.off_hsplit = o;
  o = align256(o + rh::HIST_BYTES * nsplit);
  l.off_crec = o;
  o = align256(o + sizeof(unsigned long long) * rh::NCH * nsplit);
  // the wide top_logprobs kernels' states, slice histograms and lists
  l.off_wide = o;
  o = align256(o + topk_wide_ws_bytes(B, V, K_max));
  l.total = o;
  return l;
}

void set_err(char** err, const std::string& msg) {
  if (!err) return;
  char* p = static_cast<char*>(std::malloc(msg.size() + 1));
  if (p) std::memcpy(p, msg.c_str(), msg.size() + 1);
  *err = p;
}

int check_shape(int B, int V, int K_max, int dtype, char** err) {
  if (dtype != MLXF_DTYPE_F32 && dtype != MLXF_DTYPE_BF16 && dtype != MLXF_DTYPE_F16) {
    set_err(err, "mlxf: dtype must be MLXF_DTYPE_F32, MLXF_DTYPE_BF16 or MLXF_DTYPE_F16");
    return MLXF_EINVAL;
  }
  if (B < 0 || B > 65535) {
    set_err(err, "mlxf: B must be in [0, 65535]");
    return MLXF_EINVAL;
  }
  if (V < 1 || V > MLXF_MAX_VOCAB) {
    set_err(err, "mlxf: V must be in [1, MLXF_MAX_VOCAB]");
    return MLXF_EINVAL;
  }
  if (K_max < 0 || K_max > MLXF_MAX_TOP_LOGPROBS) {
    set_err(err, "mlxf: K_max must be in [0, MLXF_MAX_TOP_LOGPROBS]");
    return MLXF_EINVAL;
  }
  return MLXF_OK;
}

// Refine stages a call needs, from host copies of the per-row parameters with
// the same sanitisation as the kernels: 0 when every row is greedy or has a
// top-k <= 63 (decided from the best-64 lists; a row whose k-th value has more
// ties than the list holds is finished by the first deciding kernel itself), 1
// when the other rows are temperature-only, else HINT_STAGES.  A null array
// reads as the sentinel (T: greedy; k: off; p: off).
//
// HINT_STAGES is 2, not NSTAGE: results are the same for every count, and the
// rows still open after a second stage are fewer than a third launch costs.
// Measured per step on MI355X, 2 vs 3 stages: B=8 V=151936 bf16 top-p 49.9 vs
// 52.6 us; B=64 V=151936 fp32 top-p 91.0 vs 94.2 us; B=256 V=262144 bf16
// mixed 161.8 vs 166.4 us (one stage: 122, 185 and 314 us).
constexpr int HINT_STAGES = 2;
int host_refine_stages(int B, int V, int dtype, const float* T, const int32_t* k, const float* p) {
  if (!T) return 0;
  auto rnd = [dtype](float x) {
    if (dtype == MLXF_DTYPE_F32) return x;
    uint32_t u;
    std::memcpy(&u, &x, 4);
    if (dtype == MLXF_DTYPE_BF16) {
      u += 0x7fffu + ((u >> 16) & 1u);
      u &= 0xffff0000u;
      float y;
      std::memcpy(&y, &u, 4);
      return y;
    }
    return static_cast<float>(static_cast<_Float16>(x));
  };
  int need = 0;
  for (int r = 0; r < B; ++r) {
    const float t = T[r];
    if (!(std::isfinite(t) && t > 0.0f && rnd(t) > 0.0f)) continue;  // greedy
    const int kk = k ? k[r] : 0;
    const float pp = p ? p[r] : 1.0f;
    const int kc = kk > 0 ? (kk < V ? kk : V) : 0;
    if (kc > 0 && kc <= KLIST_MAX) continue;
    if (kc == 0 && !(pp > 0.0f && pp < 1.0f)) {
      need = need > 1 ? need : 1;
      continue;
    }
    return HINT_STAGES;
  }
  return need;
}


int run_sample(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
               const float* d_temperature, const int32_t* d_top_k, const float* d_top_p, const float* d_min_p,
               const int32_t* d_top_logprobs, const float* d_uniforms, int32_t* d_out_ids,
               float* d_out_logprobs, int32_t* d_out_top_ids, float* d_out_top_logprobs,
               int K_max, void* d_workspace, size_t workspace_bytes, void* stream, int nst, char** err) {
  try {
    int rc = check_shape(B, V, K_max, dtype, err);
    if (rc) return rc;
    if (B == 0) return MLXF_OK;
    if (!d_logits || !d_out_ids) {
      set_err(err, "mlxf: d_logits and d_out_ids must not be NULL");
      return MLXF_EINVAL;
    }
    if (row_stride < V) {
      set_err(err, "mlxf: row_stride must be >= V");
      return MLXF_EINVAL;
    }
    if (d_temperature && !d_uniforms) {
      set_err(err, "mlxf: d_uniforms is required when d_temperature is given");
      return MLXF_EINVAL;
    }
    if (K_max > 0 && (!d_out_top_ids || !d_out_top_logprobs)) {
      set_err(err, "mlxf: K_max > 0 needs d_out_top_ids and d_out_top_logprobs");
      return MLXF_EINVAL;
    }
    const Layout l = make_layout(B, V, K_max, dtype);
    if (!d_workspace || workspace_bytes < l.total) {
      set_err(err, "mlxf: workspace is NULL or smaller than mlxf_sampler_workspace_size()");
      return MLXF_EWORKSPACE;
    }
    if (reinterpret_cast<uintptr_t>(d_workspace) & 255u) {
      set_err(err, "mlxf: workspace must be 256-byte aligned");
      return MLXF_EINVAL;
    }
    const size_t esz = dtype == MLXF_DTYPE_F32 ? 4 : 2;
    if (reinterpret_cast<uintptr_t>(d_logits) % esz) {
      set_err(err, "mlxf: d_logits is not aligned to its element size");
      return MLXF_EINVAL;
    }
    const bool vecok = (reinterpret_cast<uintptr_t>(d_logits) % 16 == 0) &&
                       ((static_cast<size_t>(row_stride) * esz) % 16 == 0);
    char* ws = static_cast<char*>(d_workspace);
    // top_logprobs wider than the sampling kernels' lists: the sampling
    // kernels run without them, then the wide kernels write every row's columns
    const bool wide = K_max > TOPK_LIST;
    const int K_main = wide ? 0 : K_max;
    Args a;
    a.logits = d_logits;
    a.row_stride = row_stride;
    a.B = B;
    a.V = V;
    a.K_max = K_main;
    a.S = l.S;
    a.L = l.L;
    a.T = d_temperature;
    a.k = d_top_k;
    a.p = d_top_p;
    a.minp = d_min_p;
    a.tlp = d_top_logprobs;
    a.u = d_uniforms;
    a.out_ids = d_out_ids;
    a.out_lp = d_out_logprobs;
    a.out_top_ids = d_out_top_ids;
    a.out_top_lp = d_out_top_logprobs;
    a.ncand = reinterpret_cast<unsigned int*>(ws + l.off_ncand);
    a.actcnt = reinterpret_cast<unsigned int*>(ws + l.off_actcnt);
    a.actlist = reinterpret_cast<unsigned int*>(ws + l.off_actlist);
    a.rec = reinterpret_cast<unsigned long long*>(ws + l.off_rec);
    a.list = reinterpret_cast<unsigned long long*>(ws + l.off_list);
    a.rowst = reinterpret_cast<unsigned long long*>(ws + l.off_rowst);
    a.hcnt = reinterpret_cast<unsigned int*>(ws + l.off_hcnt);
    a.hmass = reinterpret_cast<unsigned long long*>(ws + l.off_hmass);
    a.above = reinterpret_cast<unsigned long long*>(ws + l.off_above);
    a.dsum = reinterpret_cast<unsigned long long*>(ws + l.off_dsum);
    a.cand = reinterpret_cast<unsigned long long*>(ws + l.off_cand);
    if (nst < -1 || nst > NSTAGE) {
      set_err(err, "mlxf: refine_stages must be in [0, 3]");
      return MLXF_EINVAL;
    }
    if (!d_temperature && nst > 0) nst = 0;  // every row greedy
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e;
    if (use_row_path(dtype, B, V, K_main, vecok, nst)) {
      RhArgs x;
      const bool split = row_split(dtype, B, V);
      x.ipc = split ? (V + ROW_CHUNK_LOGITS - 1) / ROW_CHUNK_LOGITS
                    : 2 * ((V + 2 * ROW_CHUNK_LOGITS - 1) / (2 * ROW_CHUNK_LOGITS));
      x.nfull = V / ROW_ITER_LOGITS;
      x.hsplit = split ? reinterpret_cast<unsigned int*>(ws + l.off_hsplit) : nullptr;
      x.crec = split ? reinterpret_cast<unsigned long long*>(ws + l.off_crec) : nullptr;
      e = launch_row16_bf16(a, l.EPT, x, st);
    } else if (dtype == MLXF_DTYPE_F32)
      e = launch_f32(a, l.EPT, vecok, nst, st);
    else if (dtype == MLXF_DTYPE_BF16)
      e = launch_bf16(a, l.EPT, vecok, nst, st);
    else
      e = launch_f16(a, l.EPT, vecok, nst, st);
    if (e == hipSuccess && wide)
      e = launch_topk_wide(d_logits, dtype, B, V, row_stride, d_top_logprobs, K_max, d_out_top_ids,
                           d_out_top_logprobs, ws + l.off_wide, st);
    if (e != hipSuccess) {
      set_err(err, std::string("mlxf: kernel launch failed: ") + hipGetErrorString(e));
      return MLXF_EHIP;
    }
    return MLXF_OK;
  } catch (...) {
    set_err(err, "mlxf: unexpected exception");
    return MLXF_EINVAL;
  }
}

// Device address of `scratch` on the GPU that runs `stream` (the current
// device for the null stream), looked up once per GPU with that GPU current.
constexpr int NOALLOC_MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[NOALLOC_MAX_DEVICES] = {};

int noalloc_scratch(void* stream, void** out, char** err) {
  int cur = 0;
  hipError_t e = hipGetDevice(&cur);
  int dev = cur;
  if (e == hipSuccess && stream) e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &dev);
  if (e != hipSuccess) {
    set_err(err, std::string("mlxf: cannot find the stream's device: ") + hipGetErrorString(e));
    return MLXF_EHIP;
  }
  if (dev < 0 || dev >= NOALLOC_MAX_DEVICES) {
    set_err(err, "mlxf: device index beyond the allocation-free entry point's table");
    return MLXF_EINVAL;
  }
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) {
      set_err(err, std::string("mlxf: hipSetDevice failed: ") + hipGetErrorString(e));
      return MLXF_EHIP;
    }
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p) {
      set_err(err, std::string("mlxf: hipGetSymbolAddress(scratch) failed: ") + hipGetErrorString(e));
      return MLXF_EHIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MLXF_OK;
}

}  // namespace
}  // namespace mlxf

using mlxf::check_shape;
using mlxf::make_layout;
using mlxf::run_sample;
using mlxf::set_err;

extern "C" {

int mlxf_sampler_abi_version(void) { return MLXF_SAMPLER_ABI_VERSION; }

void mlxf_string_free(char* s) { std::free(s); }

int mlxf_sampler_workspace_size(int B, int V, int K_max, int dtype, size_t* bytes, char** err) {
  try {
    const int rc = check_shape(B, V, K_max, dtype, err);
    if (rc) return rc;
    if (!bytes) {
      set_err(err, "mlxf: bytes must not be NULL");
      return MLXF_EINVAL;
    }
    *bytes = make_layout(B, V, K_max, dtype).total;
    return MLXF_OK;
  } catch (...) {
    set_err(err, "mlxf: unexpected exception");
    return MLXF_EINVAL;
  }
}

int mlxf_sampler_workspace_init(void* d_workspace, size_t workspace_bytes, void* stream,
                                char** err) {
  if (!d_workspace || (reinterpret_cast<uintptr_t>(d_workspace) & 255u)) {
    set_err(err, "mlxf: workspace must be non-NULL and 256-byte aligned");
    return MLXF_EINVAL;
  }
  const size_t bytes = workspace_bytes < mlxf::CTR_BYTES_MAX ? workspace_bytes : mlxf::CTR_BYTES_MAX;
  const size_t n = bytes / sizeof(unsigned int);
  if (n == 0) return MLXF_OK;
  hipLaunchKernelGGL(mlxf::k_zero, dim3(static_cast<unsigned int>((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), static_cast<unsigned int*>(d_workspace), n);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_err(err, std::string("mlxf: kernel launch failed: ") + hipGetErrorString(e));
    return MLXF_EHIP;
  }
  return MLXF_OK;
}

int mlxf_sample(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                const int32_t* d_top_logprobs, const float* d_uniforms, int32_t* d_out_ids,
                float* d_out_logprobs, int32_t* d_out_top_ids, float* d_out_top_logprobs,
                int K_max, void* d_workspace, size_t workspace_bytes, void* stream, char** err) {
  return run_sample(d_logits, dtype, B, V, row_stride, d_temperature, d_top_k, d_top_p, nullptr,
                    d_top_logprobs, d_uniforms, d_out_ids, d_out_logprobs, d_out_top_ids,
                    d_out_top_logprobs, K_max, d_workspace, workspace_bytes, stream, mlxf::HINT_STAGES, err);
}

int mlxf_sample_staged(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                       const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                       const int32_t* d_top_logprobs, const float* d_uniforms, int32_t* d_out_ids,
                       float* d_out_logprobs, int32_t* d_out_top_ids, float* d_out_top_logprobs,
                       int K_max, void* d_workspace, size_t workspace_bytes, int refine_stages,
                       void* stream, char** err) {
  if (refine_stages < 0) {
    set_err(err, "mlxf: refine_stages must be in [0, 3]");
    return MLXF_EINVAL;
  }
  return run_sample(d_logits, dtype, B, V, row_stride, d_temperature, d_top_k, d_top_p, nullptr,
                    d_top_logprobs, d_uniforms, d_out_ids, d_out_logprobs, d_out_top_ids,
                    d_out_top_logprobs, K_max, d_workspace, workspace_bytes, stream, refine_stages, err);
}

int mlxf_sample_ex(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                   const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                   const float* d_min_p, const int32_t* d_top_logprobs, const float* d_uniforms,
                   int32_t* d_out_ids, float* d_out_logprobs, int32_t* d_out_top_ids,
                   float* d_out_top_logprobs, int K_max, void* d_workspace, size_t workspace_bytes,
                   int refine_stages, void* stream, char** err) {
  if (refine_stages < 0) {
    set_err(err, "mlxf: refine_stages must be in [0, 3]");
    return MLXF_EINVAL;
  }
  return run_sample(d_logits, dtype, B, V, row_stride, d_temperature, d_top_k, d_top_p, d_min_p,
                    d_top_logprobs, d_uniforms, d_out_ids, d_out_logprobs, d_out_top_ids,
                    d_out_top_logprobs, K_max, d_workspace, workspace_bytes, stream, refine_stages, err);
}

int mlxf_sample_noalloc(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                        const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                        const float* d_min_p, const int32_t* d_top_logprobs, const float* d_uniforms,
                        int32_t* d_out_ids, float* d_out_logprobs, int32_t* d_out_top_ids,
                        float* d_out_top_logprobs, int K_max, int refine_stages, void* stream,
                        char** err) {
  try {
    if (refine_stages < 0) {
      set_err(err, "mlxf: refine_stages must be in [0, 3]");
      return MLXF_EINVAL;
    }
    int rc = check_shape(B, V, K_max, dtype, err);
    if (rc) return rc;
    const size_t need = make_layout(B, V, K_max, dtype).total;
    if (need > MLXF_NOALLOC_SCRATCH_BYTES) {
      set_err(err, "mlxf: mlxf_sample_noalloc: this shape needs " + std::to_string(need) +
                       " bytes of scratch, more than its fixed " +
                       std::to_string(static_cast<size_t>(MLXF_NOALLOC_SCRATCH_BYTES)) +
                       "; use mlxf_sample_ex with a workspace");
      return MLXF_EWORKSPACE;
    }
    if (B == 0) return MLXF_OK;
    void* ws = nullptr;
    rc = mlxf::noalloc_scratch(stream, &ws, err);
    if (rc) return rc;
    return run_sample(d_logits, dtype, B, V, row_stride, d_temperature, d_top_k, d_top_p, d_min_p,
                      d_top_logprobs, d_uniforms, d_out_ids, d_out_logprobs, d_out_top_ids,
                      d_out_top_logprobs, K_max, ws, MLXF_NOALLOC_SCRATCH_BYTES, stream, refine_stages,
                      err);
  } catch (...) {
    set_err(err, "mlxf: unexpected exception");
    return MLXF_EINVAL;
  }
}

int mlxf_sampler_first_pass(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                            const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                            const int32_t* d_top_logprobs, const float* d_uniforms, int32_t* d_out_ids,
                            float* d_out_logprobs, int32_t* d_out_top_ids, float* d_out_top_logprobs,
                            int K_max, void* d_workspace, size_t workspace_bytes, void* stream, char** err) {
  return run_sample(d_logits, dtype, B, V, row_stride, d_temperature, d_top_k, d_top_p, nullptr,
                    d_top_logprobs, d_uniforms, d_out_ids, d_out_logprobs, d_out_top_ids,
                    d_out_top_logprobs, K_max, d_workspace, workspace_bytes, stream, -1, err);
}

int mlxf_sampler_refine_stages(int B, int V, int dtype, const float* h_temperature,
                               const int32_t* h_top_k, const float* h_top_p) {
  return mlxf::host_refine_stages(B, V, dtype, h_temperature, h_top_k, h_top_p);
}

int mlxf_greedy(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                int32_t* d_out_ids, void* d_workspace, size_t workspace_bytes, void* stream,
                char** err) {
  return run_sample(d_logits, dtype, B, V, row_stride, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                    d_out_ids, nullptr, nullptr, nullptr, 0, d_workspace, workspace_bytes, stream, 0,
                    err);
}

}  // extern "C"
