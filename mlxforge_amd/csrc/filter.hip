// filter.hip -- the reference's filter helpers as calls of their own:
// Sampler::apply_top_k / apply_top_p / apply_min_p (src/sample/sampler.h:63-69,
// src/sample/sampler.cpp:63-93), each writing the logits with every removed
// entry set to -inf, and their composition after the temperature division in
// the order Sampler::sample applies them (src/sample/sampler.cpp:158-163).
// The kept sets are the sampling call's (the same z' = round_dtype(z / T), the
// same exact fixed-point masses for the nucleus, ties at the top-k threshold
// kept, the nucleus's partial tie group kept by index order, min_p against the
// max's own weight), so a filter followed by a plain draw keeps what the
// sampling call keeps.
//
// One 1024-thread workgroup per row.  The first pass writes z' into the
// output row, which then serves as the row's scratch: the top-k threshold and
// the nucleus cutoff are radix selections over 32-bit order keys (four 8-bit
// digit levels, a histogram of counts or of masses in LDS per level), and the
// last pass writes -inf over the removed entries.  The row is read about a
// dozen times, which suits a helper the decode step never calls.
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <string>

#include "sampler_impl.hpp"

namespace mlxf {
namespace {

constexpr int FT = 1024;      // threads per workgroup
constexpr int FW = FT / 64;   // waves

struct FArgs {
  const void* logits;
  long long row_stride;
  void* out;
  long long out_stride;
  int B, V;
  // per-row arrays (NULL: the scalar below for every row)
  const float* T;
  const int* k;
  const float* p;
  const float* minp;
  float Ts, ps, mps;
  int ks;
};

struct FLds {
  unsigned int hc[256];
  unsigned long long hm[256];
  unsigned long long u64r[FW];
  float fr[FW];
  int ir[FW];
  unsigned int sel[4];
  unsigned long long sel64[2];
};

template <int DT>
__device__ __forceinline__ void st1(void* row, int i, float v) {
  if constexpr (DT == MLXF_DTYPE_F32) {
    static_cast<float*>(row)[i] = v;
  } else if constexpr (DT == MLXF_DTYPE_BF16) {
    static_cast<unsigned short*>(row)[i] = static_cast<unsigned short>(__float_as_uint(v) >> 16);
  } else {
    static_cast<__half*>(row)[i] = __float2half_rn(v);
  }
}
// The stored value, NaN kept as NaN (the first pass has already read NaN as
// -inf and written that).
template <int DT>
__device__ __forceinline__ float raw1(const void* row, int i) {
  if constexpr (DT == MLXF_DTYPE_F32) {
    return static_cast<const float*>(row)[i];
  } else if constexpr (DT == MLXF_DTYPE_BF16) {
    return __uint_as_float(static_cast<unsigned int>(static_cast<const unsigned short*>(row)[i]) << 16);
  } else {
    return __half2float(static_cast<const __half*>(row)[i]);
  }
}

// Order key of a stored z': -0 and +0 compare equal (as the reference's float
// comparisons do), so they share a key.
__device__ __forceinline__ unsigned int okey(float zp) { return f2key(zp + 0.0f); }

template <typename T>
__device__ __forceinline__ T fsum(T x, T* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  x = wave_sum(x);
  __syncthreads();
  if (lane == 0) red[wid] = x;
  __syncthreads();
  return rdl(row_sum16(lane < FW ? red[lane & (FW - 1)] : T(0)), 0);
}

// Radix selection over the order keys of the row's candidates (elements whose
// key passes `in`): the key c such that the measure (count, or fixed-point
// mass when MASS) of candidates with key > c is below `target` and with key
// >= c reaches it.  Returns c; *above = the measure above c, *cnt = the
// number of candidates with key c.
template <bool MASS, typename Load, typename In, typename Mass>
__device__ unsigned int radix_select(int V, unsigned long long target, Load load, In in, Mass massf, FLds& sh,
                                     unsigned long long* above, unsigned int* cnt) {
  const int tid = threadIdx.x;
  unsigned int prefix = 0u, mask = 0u;
  unsigned long long rem = target, abv = 0ull;
  unsigned int c_at = 0u;
  for (int shift = 24; shift >= 0; shift -= 8) {
    __syncthreads();
    if (tid < 256) {
      sh.hc[tid] = 0u;
      sh.hm[tid] = 0ull;
    }
    if (tid == 0) {
      sh.sel[0] = 0u;
      sh.sel[1] = 0u;
      sh.sel64[0] = 0ull;
    }
    __syncthreads();
    for (int i = tid; i < V; i += FT) {
      const float zp = load(i);
      const unsigned int key = okey(zp);
      if ((key & mask) == prefix && in(zp, key)) {
        const unsigned int d = (key >> shift) & 255u;
        __hip_atomic_fetch_add(&sh.hc[d], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        if (MASS) {
          const unsigned long long m = massf(zp);
          if (m) __hip_atomic_fetch_add(&sh.hm[d], m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        }
      }
    }
    __syncthreads();
    // digits in descending order: thread t < 256 takes digit 255 - t
    const unsigned int d = 255u - static_cast<unsigned int>(tid & 255);
    const unsigned long long meas = tid < 256 ? (MASS ? sh.hm[d] : static_cast<unsigned long long>(sh.hc[d])) : 0ull;
    unsigned long long tot;
    const unsigned long long excl = rh::bscan(meas, sh.u64r, &tot);
    if (tid < 256 && excl < rem && rem <= excl + meas) {
      sh.sel[0] = d;
      sh.sel64[0] = excl;
      sh.sel[1] = sh.hc[d];
    }
    __syncthreads();
    const unsigned int dd = sh.sel[0];
    const unsigned long long ex = sh.sel64[0];
    c_at = sh.sel[1];
    rem -= ex;
    abv += ex;
    prefix |= dd << shift;
    mask |= 255u << shift;
  }
  *above = abv;
  *cnt = c_at;
  return prefix;
}

template <int DT>
__global__ __launch_bounds__(FT, 1) void k_filter(FArgs f) {
  __shared__ FLds sh;
  const int tid = threadIdx.x;
  const int r = static_cast<int>(blockIdx.x);
  const int V = f.V;
  const void* irow = static_cast<const char*>(f.logits) + static_cast<size_t>(r) * f.row_stride * elem_size<DT>();
  void* orow = static_cast<char*>(f.out) + static_cast<size_t>(r) * f.out_stride * elem_size<DT>();

  // ---- the row's parameters (the sampling call's sentinels)
  const float T = f.T ? f.T[r] : f.Ts;
  const float Tr = round_dt<DT>(T);
  const bool div = __builtin_isfinite(T) && T > 0.0f && Tr > 0.0f;
  const int k0 = f.k ? f.k[r] : f.ks;
  const int kk = k0 > 0 ? (k0 < V ? k0 : V) : 0;
  // (a p that rounds to 1 in the dtype keeps every element: every prior mass
  // is below the whole mass.  With integer masses the elements of zero mass
  // would reach it, so the filter is off then.)
  const float p = f.p ? f.p[r] : f.ps;
  const float pr = round_dt<DT>(p);
  const bool topp = p > 0.0f && p < 1.0f && pr < 1.0f;
  const float mp = f.minp ? f.minp[r] : f.mps;
  const float mr = (mp > 0.0f && mp <= 1.0f) ? round_dt<DT>(mp) : 0.0f;

  // ---- pass 1: z' into the output row (NaN read as -inf), and the row max
  float mx = -INFINITY;
  for (int i = tid; i < V; i += FT) {
    const float z = ld1<DT>(irow, i);
    const float zp = div ? round_dt<DT>(z / Tr) : z;
    st1<DT>(orow, i, zp);
    mx = fmaxf(mx, zp);
  }
  float Mp;
  {
    const float w = wave_max(mx);
    if ((tid & 63) == 0) sh.fr[tid >> 6] = w;
    // the stores above are complete before the barrier, and stale L1 lines
    // (the row itself when filtering in place) are dropped after it: the
    // passes below read the output row back
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    Mp = rdl(row_max16(sh.fr[tid & (FW - 1)]), 0);
  }
  if (Mp == -INFINITY || (kk == 0 && !topp && mr == 0.0f)) return;  // nothing is removed
  const bool minf = Mp == INFINITY;
  const float nc = minf ? 0.0f : -(Mp * LOG2E);
  auto massf = [&](float zp) -> unsigned long long { return q40(wfun(zp + 0.0f, Mp, nc, minf)); };
  auto zload = [&](int i) { return raw1<DT>(orow, i); };

  // ---- top-k: the k'-th largest key counting multiplicity; every element at
  // or above it is kept (src/sample/sampler.cpp:63-68)
  unsigned int tk = 0u;
  if (kk > 0 && kk < V) {
    unsigned long long ab;
    unsigned int c;
    tk = radix_select<false>(V, static_cast<unsigned long long>(kk), zload,
                             [](float, unsigned int) { return true; }, massf, sh, &ab, &c);
  }

  // ---- top-p over the top-k survivors (src/sample/sampler.cpp:70-85): keep
  // while the mass before an element, in (z' desc, index asc) order, is below
  // ceil(p * W); the cutoff key's tie group keeps its first t in index order
  unsigned int ck = 0u;          // keys above ck: kept; key ck: the first tkeep
  unsigned int tkeep = 0xffffffffu;
  if (topp) {
    unsigned long long ms = 0ull;
    for (int i = tid; i < V; i += FT) {
      const float zp = raw1<DT>(orow, i);
      if (okey(zp) >= tk) ms += massf(zp);
    }
    const unsigned long long W = fsum(ms, sh.u64r);
    unsigned long long PW = static_cast<unsigned long long>(ceil(static_cast<double>(pr) * static_cast<double>(W)));
    if (PW < 1ull) PW = 1ull;
    unsigned long long above;
    unsigned int g;
    ck = radix_select<true>(V, PW, zload, [tk](float, unsigned int key) { return key >= tk; }, massf, sh, &above,
                            &g);
    const unsigned long long wt = massf(key2f(ck));
    const unsigned int t = ties_kept(PW > above ? PW - above : 0ull, wt, g);
    tkeep = t >= g ? 0xffffffffu : t;
  }
  // ---- min_p after them (src/sample/sampler.cpp:87-93): the weights that
  // reach min_p times the max's own weight
  const float thr = mr > 0.0f ? minp_thr(mr, Mp, nc, minf) : 0.0f;

  // ---- the last pass: -inf over every removed entry.  The partial tie group
  // needs index order: thread t takes the contiguous range [t E, (t + 1) E)
  const int E = (V + FT - 1) / FT;
  const int i0 = min(tid * E, V), i1 = min(i0 + E, V);
  unsigned int rank = 0u;
  if (tkeep != 0xffffffffu) {
    int mine = 0;
    for (int i = i0; i < i1; ++i) mine += okey(raw1<DT>(orow, i)) == ck ? 1 : 0;
    int tot;
    rank = static_cast<unsigned int>(rh::bscan(mine, sh.ir, &tot));
  }
  for (int i = i0; i < i1; ++i) {
    const float zp = raw1<DT>(orow, i);
    const unsigned int key = okey(zp);
    bool keep = key >= tk;
    if (topp) {
      if (key < ck) {
        keep = false;
      } else if (key == ck && tkeep != 0xffffffffu) {
        keep = keep && rank < tkeep;
        ++rank;
      }
    }
    if (mr > 0.0f) keep = keep && wfun(zp + 0.0f, Mp, nc, minf) >= thr;
    if (!keep && zp != -INFINITY) st1<DT>(orow, i, -INFINITY);
  }
}

// ---------------------------------------------------------------------------
// top_logprobs wider than the sampling kernels' best-64 lists (64 < K <= 4096):
// top_k_logprobs (src/sample/sampler.cpp:30-38; K = min(top_logprobs, V) at
// :52) as a call of its own after the sampling kernels.  One 1024-thread
// workgroup per row: the log-sum-exp of the unscaled row (fp64 partials), the
// K-th largest logit by a radix selection, the K entries (every logit above
// it, then the tied ones in index order) gathered into LDS and sorted by
// (logit desc, index asc) with a bitonic network, then written as (id, logit
// - LSE); columns past the row's K get id -1 and -inf.

constexpr int TOPK_WIDE_MAX = 4096;

struct TkLds {
  FLds f;
  unsigned long long ent[TOPK_WIDE_MAX];  // (key << 32) | ~index: one unsigned order, larger first
  unsigned int n;
  double dr[FW];
};

template <int DT>
__global__ __launch_bounds__(FT, 1) void k_topk_wide(const void* logits, long long row_stride, int V, const int* tlp,
                                                     int K_max, int* top_ids, float* top_lp) {
  __shared__ TkLds sh;
  const int tid = threadIdx.x;
  const int r = static_cast<int>(blockIdx.x);
  const void* row = static_cast<const char*>(logits) + static_cast<size_t>(r) * row_stride * elem_size<DT>();
  int* oid = top_ids + static_cast<size_t>(r) * K_max;
  float* olp = top_lp + static_cast<size_t>(r) * K_max;
  const int t = tlp ? tlp[r] : -1;
  const int K = t > 0 ? min(min(t, K_max), V) : 0;
  for (int j = K + tid; j < K_max; j += FT) {
    oid[j] = -1;
    olp[j] = -INFINITY;
  }
  if (K == 0) return;
  auto load = [&](int i) { return ld1<DT>(row, i); };  // NaN reads as -inf

  // ---- log-sum-exp of the unscaled row
  float mx = -INFINITY;
  for (int i = tid; i < V; i += FT) mx = fmaxf(mx, load(i));
  float M;
  {
    const float w = wave_max(mx);
    if ((tid & 63) == 0) sh.f.fr[tid >> 6] = w;
    __syncthreads();
    M = rdl(row_max16(sh.f.fr[tid & (FW - 1)]), 0);
  }
  double part = 0.0;
  for (int i = tid; i < V; i += FT) part += wexp_d(load(i), M);
  const double lse = static_cast<double>(M) + log(fsum(part, sh.dr));

  // ---- the K-th largest logit (counting multiplicity) and the entries
  unsigned long long above;
  unsigned int g;
  const unsigned int tau = radix_select<false>(V, static_cast<unsigned long long>(K), load,
                                               [](float, unsigned int) { return true; },
                                               [](float) { return 0ull; }, sh.f, &above, &g);
  const unsigned int need_eq = static_cast<unsigned int>(K) - static_cast<unsigned int>(above);
  // contiguous ranges (index order for the tied entries)
  const int E = (V + FT - 1) / FT;
  const int i0 = min(tid * E, V), i1 = min(i0 + E, V);
  int mine = 0;
  for (int i = i0; i < i1; ++i) mine += okey(load(i)) == tau ? 1 : 0;
  int tot;
  unsigned int rank = static_cast<unsigned int>(rh::bscan(mine, sh.f.ir, &tot));
  if (tid == 0) sh.n = 0u;
  __syncthreads();
  for (int i = i0; i < i1; ++i) {
    const unsigned int key = okey(load(i));
    bool take = key > tau;
    if (key == tau) {
      take = rank < need_eq;
      ++rank;
    }
    if (take) {
      const unsigned int slot = __hip_atomic_fetch_add(&sh.n, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (slot < static_cast<unsigned int>(TOPK_WIDE_MAX))
        sh.ent[slot] = (static_cast<unsigned long long>(key) << 32) | (0xffffffffu - static_cast<unsigned int>(i));
    }
  }
  __syncthreads();
  // ---- bitonic sort, descending, over the next power of two (padding: 0)
  int np = 1;
  while (np < K) np <<= 1;
  for (int j = K + tid; j < np; j += FT) sh.ent[j] = 0ull;
  __syncthreads();
  for (int k = 2; k <= np; k <<= 1) {
    for (int jj = k >> 1; jj > 0; jj >>= 1) {
      for (int i = tid; i < np; i += FT) {
        const int ixj = i ^ jj;
        if (ixj > i) {
          const unsigned long long a = sh.ent[i], b = sh.ent[ixj];
          const bool desc = (i & k) == 0;
          if (desc ? (a < b) : (a > b)) {
            sh.ent[i] = b;
            sh.ent[ixj] = a;
          }
        }
      }
      __syncthreads();
    }
  }
  // ---- write (id, logit - LSE)
  for (int j = tid; j < K; j += FT) {
    const unsigned long long e = sh.ent[j];
    const int id = static_cast<int>(0xffffffffu - static_cast<unsigned int>(e));
    oid[j] = id;
    olp[j] = static_cast<float>(static_cast<double>(load(id)) - lse);
  }
}

void set_err(char** err, const std::string& msg) {
  if (!err) return;
  char* q = static_cast<char*>(std::malloc(msg.size() + 1));
  if (q) std::memcpy(q, msg.c_str(), msg.size() + 1);
  *err = q;
}

int launch_filter(const void* d_logits, int dtype, int B, int V, int64_t row_stride, void* d_out, int64_t out_stride,
                  FArgs f, void* stream, char** err) {
  if (dtype != MLXF_DTYPE_F32 && dtype != MLXF_DTYPE_BF16 && dtype != MLXF_DTYPE_F16) {
    set_err(err, "mlxf: dtype must be MLXF_DTYPE_F32, MLXF_DTYPE_BF16 or MLXF_DTYPE_F16");
    return MLXF_EINVAL;
  }
  if (B < 0 || V < 1 || V > MLXF_MAX_VOCAB || row_stride < V || out_stride < V) {
    set_err(err, "mlxf: bad shape (B >= 0, V in [1, MLXF_MAX_VOCAB], row_stride and out_stride >= V)");
    return MLXF_EINVAL;
  }
  if (B == 0) return MLXF_OK;
  if (!d_logits || !d_out) {
    set_err(err, "mlxf: d_logits and d_out must not be NULL");
    return MLXF_EINVAL;
  }
  const size_t esz = dtype == MLXF_DTYPE_F32 ? 4 : 2;
  if ((reinterpret_cast<uintptr_t>(d_logits) % esz) || (reinterpret_cast<uintptr_t>(d_out) % esz)) {
    set_err(err, "mlxf: d_logits or d_out is not aligned to its element size");
    return MLXF_EINVAL;
  }
  if (d_out != d_logits || out_stride != row_stride) {
    // rows that overlap without being the same row would be read after
    // being written
    const char* a0 = static_cast<const char*>(d_logits);
    const char* a1 = a0 + (static_cast<size_t>(B - 1) * row_stride + V) * esz;
    const char* b0 = static_cast<const char*>(d_out);
    const char* b1 = b0 + (static_cast<size_t>(B - 1) * out_stride + V) * esz;
    if (a0 < b1 && b0 < a1) {
      set_err(err, "mlxf: d_out overlaps d_logits without being the same rows (in place: d_out == d_logits, "
                   "out_stride == row_stride)");
      return MLXF_EINVAL;
    }
  }
  f.logits = d_logits;
  f.row_stride = row_stride;
  f.out = d_out;
  f.out_stride = out_stride;
  f.B = B;
  f.V = V;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned int>(B)), block(FT);
  if (dtype == MLXF_DTYPE_F32)
    hipLaunchKernelGGL(k_filter<MLXF_DTYPE_F32>, grid, block, 0, st, f);
  else if (dtype == MLXF_DTYPE_BF16)
    hipLaunchKernelGGL(k_filter<MLXF_DTYPE_BF16>, grid, block, 0, st, f);
  else
    hipLaunchKernelGGL(k_filter<MLXF_DTYPE_F16>, grid, block, 0, st, f);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_err(err, std::string("mlxf: kernel launch failed: ") + hipGetErrorString(e));
    return MLXF_EHIP;
  }
  return MLXF_OK;
}

FArgs scalars(float T, int k, float p, float mp) {
  FArgs f{};
  f.Ts = T;
  f.ks = k;
  f.ps = p;
  f.mps = mp;
  return f;
}

}  // namespace

hipError_t launch_topk_wide(const void* logits, int dtype, int B, int V, long long row_stride, const int* tlp,
                            int K_max, int* top_ids, float* top_lp, hipStream_t st) {
  const dim3 grid(static_cast<unsigned int>(B)), block(FT);
  if (dtype == MLXF_DTYPE_F32)
    hipLaunchKernelGGL(k_topk_wide<MLXF_DTYPE_F32>, grid, block, 0, st, logits, row_stride, V, tlp, K_max, top_ids,
                       top_lp);
  else if (dtype == MLXF_DTYPE_BF16)
    hipLaunchKernelGGL(k_topk_wide<MLXF_DTYPE_BF16>, grid, block, 0, st, logits, row_stride, V, tlp, K_max, top_ids,
                       top_lp);
  else
    hipLaunchKernelGGL(k_topk_wide<MLXF_DTYPE_F16>, grid, block, 0, st, logits, row_stride, V, tlp, K_max, top_ids,
                       top_lp);
  return hipGetLastError();
}

}  // namespace mlxf

extern "C" int mlxf_filter_logits(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                                  const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                                  const float* d_min_p, void* d_out, int64_t out_stride, void* stream, char** err) {
  try {
    mlxf::FArgs f = mlxf::scalars(0.0f, 0, 1.0f, 0.0f);
    f.T = d_temperature;
    f.k = d_top_k;
    f.p = d_top_p;
    f.minp = d_min_p;
    return mlxf::launch_filter(d_logits, dtype, B, V, row_stride, d_out, out_stride, f, stream, err);
  } catch (...) {
    mlxf::set_err(err, "mlxf: unexpected exception");
    return MLXF_EINVAL;
  }
}

extern "C" int mlxf_apply_top_k(const void* d_logits, int dtype, int B, int V, int64_t row_stride, int k,
                                void* d_out, int64_t out_stride, void* stream, char** err) {
  return mlxf::launch_filter(d_logits, dtype, B, V, row_stride, d_out, out_stride, mlxf::scalars(0.0f, k, 1.0f, 0.0f),
                             stream, err);
}

extern "C" int mlxf_apply_top_p(const void* d_logits, int dtype, int B, int V, int64_t row_stride, float p,
                                void* d_out, int64_t out_stride, void* stream, char** err) {
  return mlxf::launch_filter(d_logits, dtype, B, V, row_stride, d_out, out_stride, mlxf::scalars(0.0f, 0, p, 0.0f),
                             stream, err);
}

extern "C" int mlxf_apply_min_p(const void* d_logits, int dtype, int B, int V, int64_t row_stride, float min_p,
                                void* d_out, int64_t out_stride, void* stream, char** err) {
  return mlxf::launch_filter(d_logits, dtype, B, V, row_stride, d_out, out_stride,
                             mlxf::scalars(0.0f, 0, 1.0f, min_p), stream, err);
}
