// sampler.hip -- MI355X (gfx950) batched token sampler behind the C ABI in
// include/mlxf_sampler.h.
//
// Replaces the per-row MLX graph of Sampler::sample (src/sample/sampler.cpp:
// 141-166) with one launch sequence over all rows of a [B, V] logits matrix.
// Each row is cut into S slices of L elements; a slice is one 256-thread
// workgroup that streams its part of the row with 16-byte loads.
//
//   k_scan    (S x B)  one HBM pass: row max / lowest-index argmax, the log-sum-
//                      exp partial, the slice's top-K by (z desc, idx asc) for
//                      top_logprobs, and -- for rows with top-k / top-p -- a
//                      2048-bin histogram (count, mass) of z' = z / T over the
//                      top 11 bits of its monotone key.
//   k_plan    (B)      combines the slices: greedy id + logprob, merged top-K,
//                      max z', and the range R of histogram bins that can hold
//                      the top-k / top-p boundary.
//   k_extract (S x B)  re-reads the slice (L2/MALL), sums the exact fixed-point
//                      mass above R and of the whole slice, and compacts the
//                      elements inside R in index order.
//   k_select  (B)      exact radix selection over the candidates: the k-th
//                      largest z' (ties kept), the nucleus cutoff (value v* and
//                      the last kept index among ties at v*), the kept mass per
//                      slice and the slice holding the draw.
//   k_draw    (B)      inverse-CDF walk of that one slice in vocabulary order.
//
// Every mass is exp(z' - max z') rounded down to a multiple of 2^-42 and summed
// as uint64, so the sums are exact, independent of summation order, and the
// draw walk sees exactly the per-slice masses k_select chose the slice with.
// There is no MFMA anywhere: nothing here is a dense contraction.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <climits>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>

#include "mlxf_sampler.h"
#include "mlxf_sampler_diag.h"

namespace {

constexpr int NB = 2048;          // histogram bins: key >> 21
constexpr int BIN_SHIFT = 21;
constexpr int SLICE_THREADS = 256;
constexpr int VEC = 8;            // elements per thread per iteration (16 B of bf16)
constexpr int ITER_ELEMS = SLICE_THREADS * VEC;
constexpr int ROW_THREADS = 1024;
constexpr int ROW_WAVES = ROW_THREADS / 64;
constexpr int TARGET_BLOCKS = 1024;  // ~4 workgroups per CU on 256 CUs
constexpr int MAX_S = 32;
constexpr int CAND_LDS = 6144;       // candidates staged in LDS by k_select
constexpr float LOG2E = 1.4426950408889634f;

enum { KIND_GREEDY = 0, KIND_TEMP = 1, KIND_HIST = 2 };

struct TopEnt {
  float v;
  int i;
};

struct SliceRec {
  float zmax;
  int zarg;
  float lse_s;  // sum exp(z - zmax) over the slice
  float pad;
};

struct SliceMass {
  unsigned long long above;  // mass of bins above R
  unsigned long long total;  // mass of the whole slice
  unsigned int ncand;
  unsigned int pad0;
  unsigned long long pad1;
};

struct RowState {
  int kind;
  int zarg;
  float zmax;
  float Mp;  // max z'
  double lse;
  int b_lo, b_hi;
  unsigned int cnt_above;
  unsigned int vkey;
  int idx_cut;
  int s_star;
  unsigned long long target_rem;
};

struct Args {
  const void* logits;
  long long row_stride;
  int B, V, K_max;
  int S, L;
  const float* T;
  const int* k;
  const float* p;
  const int* tlp;
  const float* u;
  int* out_ids;
  float* out_lp;
  int* out_top_ids;
  float* out_top_lp;
  // workspace views
  RowState* rs;
  SliceRec* rec;
  TopEnt* top;
  unsigned int* hcnt;
  unsigned long long* hmass;
  SliceMass* sm;
  uint2* cand;
};

// ---------------------------------------------------------------- helpers --

__device__ __forceinline__ unsigned int f2key(float f) {
  unsigned int u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key2f(unsigned int k) {
  unsigned int u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// Round-to-nearest-even into the logits dtype (the dtype-faithful temperature
// division of src/sample/sampler.cpp:158).
template <int DT>
__device__ __forceinline__ float round_dt(float x) {
  if constexpr (DT == MLXF_DTYPE_BF16) {
    unsigned int u = __float_as_uint(x);
    u += 0x7fffu + ((u >> 16) & 1u);
    return __uint_as_float(u & 0xffff0000u);
  } else if constexpr (DT == MLXF_DTYPE_F16) {
    return __half2float(__float2half_rn(x));
  } else {
    return x;
  }
}

template <int DT>
constexpr int elem_size() {
  return DT == MLXF_DTYPE_F32 ? 4 : 2;
}

template <int DT>
__device__ __forceinline__ float ld1(const void* row, int i) {
  float v;
  if constexpr (DT == MLXF_DTYPE_F32) {
    v = static_cast<const float*>(row)[i];
  } else if constexpr (DT == MLXF_DTYPE_BF16) {
    v = __uint_as_float(static_cast<unsigned int>(static_cast<const unsigned short*>(row)[i]) << 16);
  } else {
    v = __half2float(static_cast<const __half*>(row)[i]);
  }
  return v != v ? -INFINITY : v;  // NaN reads as -inf
}

// 8 consecutive elements starting at i0 (i0 % 8 == 0); entries past `end` are
// -inf and *nv counts the valid ones.
template <int DT, bool VECOK>
__device__ __forceinline__ void load8(const void* row, int i0, int end, float (&v)[VEC], int& nv) {
  nv = end - i0;
  nv = nv < 0 ? 0 : (nv > VEC ? VEC : nv);
  if (VECOK && nv == VEC) {
    if constexpr (DT == MLXF_DTYPE_F32) {
      const float4* p = reinterpret_cast<const float4*>(static_cast<const float*>(row) + i0);
      float4 a = p[0], b = p[1];
      v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
      v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
      uint4 q = *reinterpret_cast<const uint4*>(static_cast<const unsigned short*>(row) + i0);
      unsigned int w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (DT == MLXF_DTYPE_BF16) {
          v[2 * j] = __uint_as_float(w[j] << 16);
          v[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        } else {
          __half_raw lo, hi;
          lo.x = static_cast<unsigned short>(w[j] & 0xffffu);
          hi.x = static_cast<unsigned short>(w[j] >> 16);
          v[2 * j] = __half2float(__half(lo));
          v[2 * j + 1] = __half2float(__half(hi));
        }
      }
    }
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[j] = v[j] != v[j] ? -INFINITY : v[j];
  } else {
#pragma unroll
    for (int j = 0; j < VEC; ++j) v[j] = j < nv ? ld1<DT>(row, i0 + j) : -INFINITY;
  }
}

// exp(x - m), with exp(m - m) = 1 also for infinite m.
__device__ __forceinline__ float wexp(float x, float m) {
  float e = __builtin_amdgcn_exp2f((x - m) * LOG2E);
  return x == m ? 1.0f : e;
}
__device__ __forceinline__ double wexp_d(float x, float m) {
  return x == m ? 1.0 : exp(static_cast<double>(x) - static_cast<double>(m));
}

// floor(w * 2^42) for w in [0, 1]: the fixed-point mass unit.
__device__ __forceinline__ unsigned long long quant(float w) {
  float t = w * 1024.0f;
  float h = floorf(t);
  float fr = t - h;
  unsigned int lo = static_cast<unsigned int>(fr * 4294967296.0f);
  unsigned int hi = static_cast<unsigned int>(h);
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) {
  return av > bv || (av == bv && ai < bi);
}

struct Mode {
  int sampling;
  float Tr;
  int kk;
  int topp;
  float pr;
  int K;
  int need_lse;
  int want_lp;
  float u;
  int kind;
};

// Per-row parameters with the reference's sentinels and the C ABI's
// sanitisation (src/sample/sampler.h:15-29, src/capi/mlxforge.cpp:43-70).
template <int DT>
__device__ __forceinline__ Mode decode(const Args& a, int r) {
  Mode m;
  const float T = a.T ? a.T[r] : 0.0f;
  m.Tr = round_dt<DT>(T);
  m.sampling = (__builtin_isfinite(T) && T > 0.0f && m.Tr > 0.0f) ? 1 : 0;
  const int k = a.k ? a.k[r] : 0;
  m.kk = (m.sampling && k > 0) ? (k < a.V ? k : a.V) : 0;
  const float p = a.p ? a.p[r] : 1.0f;
  m.topp = (m.sampling && p > 0.0f && p < 1.0f) ? 1 : 0;
  m.pr = round_dt<DT>(p);
  const int tlp = a.tlp ? a.tlp[r] : -1;
  int K = tlp > 0 ? tlp : 0;
  K = K < a.K_max ? K : a.K_max;
  K = K < a.V ? K : a.V;
  m.K = K;
  m.want_lp = (a.out_lp != nullptr && tlp >= 0) ? 1 : 0;
  m.need_lse = (tlp >= 0 && (a.out_lp != nullptr || K > 0)) ? 1 : 0;
  float u = a.u ? a.u[r] : 0.0f;
  if (!(u >= 0.0f)) u = 0.0f;
  if (u >= 1.0f) u = 0x1.fffffep-1f;
  m.u = u;
  m.kind = !m.sampling ? KIND_GREEDY : ((m.kk > 0 || m.topp) ? KIND_HIST : KIND_TEMP);
  return m;
}

template <int DT>
__device__ __forceinline__ const void* row_ptr(const Args& a, int r) {
  return static_cast<const char*>(a.logits) +
         static_cast<size_t>(r) * static_cast<size_t>(a.row_stride) * elem_size<DT>();
}

// Bitonic sort of one entry per lane, best (v desc, i asc) in lane 0.
__device__ __forceinline__ void wave_sort(float& v, int& i) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      float ov = __shfl_xor(v, j, 64);
      int oi = __shfl_xor(i, j, 64);
      const bool first = (lane & j) == 0;
      const bool asc = (lane & k) == 0;
      const bool ob = better(ov, oi, v, i);
      const bool take = (first == asc) ? ob : !ob;
      if (take) {
        v = ov;
        i = oi;
      }
    }
  }
}

// Final bitonic merge stage (k = 64) of a bitonic lane sequence.
__device__ __forceinline__ void wave_merge(float& v, int& i) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int j = 32; j > 0; j >>= 1) {
    float ov = __shfl_xor(v, j, 64);
    int oi = __shfl_xor(i, j, 64);
    const bool first = (lane & j) == 0;
    const bool ob = better(ov, oi, v, i);
    const bool take = first ? ob : !ob;
    if (take) {
      v = ov;
      i = oi;
    }
  }
}

// (lv, li): sorted top-64 list of the wave.  Merge a sorted list (nv, ni).
__device__ __forceinline__ void wave_list_merge(float& lv, int& li, float nv, int ni) {
  const int lane = threadIdx.x & 63;
  float rv = __shfl(nv, 63 - lane, 64);
  int ri = __shfl(ni, 63 - lane, 64);
  if (better(rv, ri, lv, li)) {
    lv = rv;
    li = ri;
  }
  wave_merge(lv, li);
}

template <typename T>
__device__ __forceinline__ T wave_sum(T x) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) x += __shfl_xor(x, o, 64);
  return x;
}

// Inclusive scan within a wave.
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T x) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    T y = __shfl_up(x, o, 64);
    if (lane >= o) x += y;
  }
  return x;
}

// Exclusive block scan (NW waves); *total gets the block sum.  Uses lds[NW+1].
template <typename T, int NW>
__device__ __forceinline__ T block_excl_scan(T x, T* lds, T* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  T inc = wave_incl_scan(x);
  __syncthreads();
  if (lane == 63) lds[wid] = inc;
  __syncthreads();
  if (wid == 0) {
    T t = lane < NW ? lds[lane] : T(0);
    T s = wave_incl_scan(t);
    if (lane < NW) lds[lane] = s - t;
    if (lane == NW - 1) lds[NW] = s;
  }
  __syncthreads();
  T res = inc - x + lds[wid];
  *total = lds[NW];
  return res;
}

template <typename T, int NW>
__device__ __forceinline__ T block_sum(T x, T* lds) {
  T tot;
  (void)block_excl_scan<T, NW>(x, lds, &tot);
  return tot;
}

// =================================================================== k_scan ==

template <int DT, bool VECOK>
__global__ __launch_bounds__(SLICE_THREADS) void k_scan(Args a) {
  __shared__ unsigned int s_cnt[NB];
  __shared__ unsigned long long s_mass[NB];
  __shared__ TopEnt s_top[4][64];
  __shared__ float s_f[8];
  __shared__ int s_i[8];
  __shared__ double s_d[8];

  const int s = blockIdx.x, r = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const Mode md = decode<DT>(a, r);
  const void* row = row_ptr<DT>(a, r);
  const int beg = s * a.L;
  const int end = min(a.V, beg + a.L);

  float bm = -INFINITY;
  int bi = INT_MAX;
  float tm = -INFINITY, ts = 0.0f;
  float lv = -INFINITY;
  int li = INT_MAX;
  float thr_v = -INFINITY;
  int thr_i = INT_MAX;

  for (int base = beg; base < end; base += ITER_ELEMS) {
    const int i0 = base + tid * VEC;
    float v[VEC];
    int nv;
    load8<DT, VECOK>(row, i0, end, v, nv);
#pragma unroll
    for (int j = 0; j < VEC; ++j)
      if (j < nv && v[j] > bm) {
        bm = v[j];
        bi = i0 + j;
      }
    if (md.need_lse) {
      float m8 = -INFINITY;
#pragma unroll
      for (int j = 0; j < VEC; ++j) m8 = fmaxf(m8, v[j]);
      if (m8 > tm) {
        ts *= wexp(tm, m8);
        tm = m8;
      }
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        if (j < nv) ts += wexp(v[j], tm);
    }
    if (md.K > 0) {
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        float ev = j < nv ? v[j] : -INFINITY;
        int ei = j < nv ? i0 + j : INT_MAX;
        const bool c = better(ev, ei, thr_v, thr_i);
        if (__ballot(c)) {
          if (!c) {
            ev = -INFINITY;
            ei = INT_MAX;
          }
          wave_sort(ev, ei);
          wave_list_merge(lv, li, ev, ei);
          thr_v = __shfl(lv, md.K - 1, 64);
          thr_i = __shfl(li, md.K - 1, 64);
        }
      }
    }
  }

  // ---- block argmax (v desc, i asc)
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    float ov = __shfl_xor(bm, o, 64);
    int oi = __shfl_xor(bi, o, 64);
    if (better(ov, oi, bm, bi)) {
      bm = ov;
      bi = oi;
    }
  }
  if (lane == 0) {
    s_f[wid] = bm;
    s_i[wid] = bi;
  }
  // ---- LSE partial
  if (md.need_lse) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      float om = __shfl_xor(tm, o, 64);
      float os = __shfl_xor(ts, o, 64);
      float nm = fmaxf(tm, om);
      ts = ts * wexp(tm, nm) + os * wexp(om, nm);
      tm = nm;
    }
    if (lane == 0) {
      s_f[4 + wid] = tm;
      s_d[wid] = ts;
    }
  }
  __syncthreads();
  float zmax = s_f[0];
  int zarg = s_i[0];
  for (int w = 1; w < 4; ++w)
    if (better(s_f[w], s_i[w], zmax, zarg)) {
      zmax = s_f[w];
      zarg = s_i[w];
    }
  if (tid == 0) {
    SliceRec rc;
    rc.zmax = zmax;
    rc.zarg = zarg;
    rc.lse_s = 0.0f;
    rc.pad = 0.0f;
    if (md.need_lse) {
      double acc = 0.0;
      for (int w = 0; w < 4; ++w) acc += s_d[w] * wexp_d(s_f[4 + w], zmax);
      rc.lse_s = static_cast<float>(acc);
    }
    a.rec[r * a.S + s] = rc;
  }

  // ---- top-K: merge the four wave lists
  if (md.K > 0) {
    s_top[wid][lane].v = lv;
    s_top[wid][lane].i = li;
    __syncthreads();
    if (wid == 0) {
      for (int w = 1; w < 4; ++w) wave_list_merge(lv, li, s_top[w][lane].v, s_top[w][lane].i);
      if (lane < md.K) {
        TopEnt e;
        e.v = lv;
        e.i = li;
        a.top[(static_cast<size_t>(r) * a.S + s) * a.K_max + lane] = e;
      }
    }
  }

  // ---- histogram of z' (count, fixed-point mass relative to the slice max z')
  if (md.kind == KIND_HIST) {
    for (int b = tid; b < NB; b += SLICE_THREADS) {
      s_cnt[b] = 0u;
      s_mass[b] = 0ull;
    }
    __syncthreads();
    const float mps = round_dt<DT>(zmax / md.Tr);
    for (int base = beg; base < end; base += ITER_ELEMS) {
      const int i0 = base + tid * VEC;
      float v[VEC];
      int nv;
      load8<DT, VECOK>(row, i0, end, v, nv);
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        if (j < nv) {
          const float zp = round_dt<DT>(v[j] / md.Tr);
          const unsigned int b = f2key(zp) >> BIN_SHIFT;
          atomicAdd(&s_cnt[b], 1u);
          const unsigned long long q = quant(wexp(zp, mps));
          if (q) atomicAdd(&s_mass[b], q);
        }
      }
    }
    __syncthreads();
    const size_t off = (static_cast<size_t>(r) * a.S + s) * NB;
    for (int b = tid; b < NB; b += SLICE_THREADS) {
      a.hcnt[off + b] = s_cnt[b];
      a.hmass[off + b] = s_mass[b];
    }
  }
}

// =================================================================== k_plan ==

template <int DT>
__global__ __launch_bounds__(ROW_THREADS) void k_plan(Args a) {
  __shared__ float s_mps[MAX_S];
  __shared__ double s_scale[MAX_S];
  __shared__ TopEnt s_top[MAX_S * 64];
  __shared__ unsigned int s_scan_u[ROW_WAVES + 1];
  __shared__ double s_scan_d[ROW_WAVES + 1];
  __shared__ int s_res[4];
  __shared__ float s_zmax;
  __shared__ int s_zarg;
  __shared__ double s_lse;

  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const Mode md = decode<DT>(a, r);
  const int S = a.S;

  // ---- combine slice records (wave 0; S <= 64)
  if (wid == 0) {
    float zm = -INFINITY;
    int za = INT_MAX;
    float ls = 0.0f;
    if (lane < S) {
      const SliceRec rc = a.rec[r * S + lane];
      zm = rc.zmax;
      za = rc.zarg;
      ls = rc.lse_s;
    }
    float bm = zm;
    int bi = za;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      float ov = __shfl_xor(bm, o, 64);
      int oi = __shfl_xor(bi, o, 64);
      if (better(ov, oi, bm, bi)) {
        bm = ov;
        bi = oi;
      }
    }
    double part = (lane < S && md.need_lse) ? static_cast<double>(ls) * wexp_d(zm, bm) : 0.0;
    part = wave_sum(part);
    if (md.sampling && lane < S) {
      const float mps = round_dt<DT>(zm / md.Tr);
      const float Mp = round_dt<DT>(bm / md.Tr);
      s_mps[lane] = mps;
      s_scale[lane] = wexp_d(mps, Mp);
    }
    if (lane == 0) {
      s_zmax = bm;
      s_zarg = bi;
      s_lse = md.need_lse ? static_cast<double>(bm) + log(part) : static_cast<double>(NAN);
    }
  }
  __syncthreads();
  const float zmax = s_zmax;
  const int zarg = s_zarg;
  const double lse = s_lse;

  if (tid == 0) {
    RowState st;
    st.kind = md.kind;
    st.zarg = zarg;
    st.zmax = zmax;
    st.Mp = md.sampling ? round_dt<DT>(zmax / md.Tr) : 0.0f;
    st.lse = lse;
    st.b_lo = NB;
    st.b_hi = -1;
    st.cnt_above = 0;
    st.vkey = 0;
    st.idx_cut = INT_MAX;
    st.s_star = 0;
    st.target_rem = 0;
    a.rs[r] = st;
    if (md.kind == KIND_GREEDY) {
      a.out_ids[r] = zarg;
      if (a.out_lp)
        a.out_lp[r] = md.want_lp ? static_cast<float>(static_cast<double>(zmax) - lse) : NAN;
    }
  }

  // ---- top_logprobs: merge the S sorted slice lists
  if (a.K_max > 0) {
    const int K = md.K;
    const int n = S * K;
    for (int e = tid; e < n; e += ROW_THREADS) s_top[e] = a.top[(static_cast<size_t>(r) * S + e / K) * a.K_max + e % K];
    __syncthreads();
    for (int e = tid; e < n; e += ROW_THREADS) {
      const TopEnt me = s_top[e];
      const int own = e / K;
      int rank = e % K;
      for (int t = 0; t < S; ++t) {
        if (t == own) continue;
        int lo = 0, hi = K;  // count entries of list t better than me
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          const TopEnt o = s_top[t * K + mid];
          if (better(o.v, o.i, me.v, me.i))
            lo = mid + 1;
          else
            hi = mid;
        }
        rank += lo;
      }
      if (rank < K && me.i < a.V) {
        a.out_top_ids[static_cast<size_t>(r) * a.K_max + rank] = me.i;
        a.out_top_lp[static_cast<size_t>(r) * a.K_max + rank] =
            static_cast<float>(static_cast<double>(me.v) - lse);
      }
    }
    for (int c = K + tid; c < a.K_max; c += ROW_THREADS) {
      a.out_top_ids[static_cast<size_t>(r) * a.K_max + c] = -1;
      a.out_top_lp[static_cast<size_t>(r) * a.K_max + c] = -INFINITY;
    }
  }

  if (md.kind != KIND_HIST) return;

  // ---- combined histogram, scanned from the top bin down
  // Thread t owns descending positions q = 2t, 2t+1 (bins NB-1-2t, NB-2-2t).
  const size_t hbase = static_cast<size_t>(r) * S * NB;
  unsigned int c[2] = {0u, 0u};
  double m[2] = {0.0, 0.0};
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int b = NB - 1 - (2 * tid + h);
    for (int t = 0; t < S; ++t) {
      c[h] += a.hcnt[hbase + static_cast<size_t>(t) * NB + b];
      m[h] += static_cast<double>(a.hmass[hbase + static_cast<size_t>(t) * NB + b]) * s_scale[t];
    }
  }
  unsigned int ctot;
  double mtot;
  const unsigned int cex = block_excl_scan<unsigned int, ROW_WAVES>(c[0] + c[1], s_scan_u, &ctot);
  const double mex = block_excl_scan<double, ROW_WAVES>(m[0] + m[1], s_scan_d, &mtot);
  const unsigned int cin[2] = {cex + c[0], cex + c[0] + c[1]};
  const double min_[2] = {mex + m[0], mex + m[0] + m[1]};
  const unsigned int cprev[2] = {cex, cin[0]};
  const double mprev[2] = {mex, min_[0]};

  if (tid == 0) {
    s_res[0] = -1;
    s_res[1] = -1;
    s_res[2] = -1;
    s_res[3] = NB;
  }
  __syncthreads();
  // top-k boundary bin: first position whose inclusive count reaches k.
  if (md.kk > 0) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
      if (cin[h] >= static_cast<unsigned int>(md.kk) && cprev[h] < static_cast<unsigned int>(md.kk))
        s_res[0] = NB - 1 - (2 * tid + h);
  }
  // lowest non-empty bin
#pragma unroll
  for (int h = 0; h < 2; ++h)
    if (c[h]) atomicMin(&s_res[3], NB - 1 - (2 * tid + h));
  __syncthreads();
  const int b_k = s_res[0];
  double W_lo = mtot, W_hi = mtot;
  if (md.kk > 0) {
    // masses strictly above and including b_k
    const int q = NB - 1 - b_k;
    if ((q >> 1) == tid) {
      const int h = q & 1;
      s_scan_d[0] = mprev[h];
      s_scan_d[1] = min_[h];
    }
    __syncthreads();
    W_lo = s_scan_d[0];
    W_hi = s_scan_d[1];
    __syncthreads();
  }
  int lo_bin, hi_bin;
  if (md.topp) {
    const double eps = 1e-5;
    const double t_hi = static_cast<double>(md.pr) * W_lo * (1.0 - eps);  // highest crossing
    const double t_lo = static_cast<double>(md.pr) * W_hi * (1.0 + eps);  // lowest crossing
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int b = NB - 1 - (2 * tid + h);
      if (min_[h] >= t_hi && (2 * tid + h == 0 || mprev[h] < t_hi)) s_res[1] = b;
      if (min_[h] >= t_lo && (2 * tid + h == 0 || mprev[h] < t_lo)) s_res[2] = b;
    }
    __syncthreads();
    int bp_hi = s_res[1] < 0 ? s_res[3] : s_res[1];
    int bp_lo = s_res[2] < 0 ? s_res[3] : s_res[2];
    if (md.kk > 0) {
      lo_bin = b_k;
      hi_bin = bp_hi > b_k ? bp_hi : b_k;
    } else {
      lo_bin = bp_lo;
      hi_bin = bp_hi;
    }
  } else {
    lo_bin = b_k;
    hi_bin = b_k;
  }
  // count strictly above hi_bin
  if (tid == 0) s_res[0] = 0;
  __syncthreads();
  {
    const int q = NB - 1 - hi_bin;
    if ((q >> 1) == tid) s_res[0] = static_cast<int>(cprev[q & 1]);
  }
  __syncthreads();
  if (tid == 0) {
    a.rs[r].b_lo = lo_bin;
    a.rs[r].b_hi = hi_bin;
    a.rs[r].cnt_above = static_cast<unsigned int>(s_res[0]);
  }
}

// ================================================================ k_extract ==

template <int DT, bool VECOK>
__global__ __launch_bounds__(SLICE_THREADS) void k_extract(Args a) {
  __shared__ int s_scan[5];
  __shared__ unsigned long long s_u64[5];

  const int s = blockIdx.x, r = blockIdx.y;
  const int tid = threadIdx.x;
  const RowState st = a.rs[r];
  if (st.kind == KIND_GREEDY) return;
  const Mode md = decode<DT>(a, r);
  const void* row = row_ptr<DT>(a, r);
  const int beg = s * a.L;
  const int end = min(a.V, beg + a.L);
  const float Mp = st.Mp;
  const unsigned int blo = static_cast<unsigned int>(st.b_lo);
  const int bhi = st.b_hi;
  uint2* cand = a.cand + (static_cast<size_t>(r) * a.S + s) * a.L;

  unsigned long long tot = 0, above = 0;
  int ncand = 0;
  for (int base = beg; base < end; base += ITER_ELEMS) {
    const int i0 = base + tid * VEC;
    float v[VEC];
    int nv;
    load8<DT, VECOK>(row, i0, end, v, nv);
    unsigned int keys[VEC];
    unsigned int cm = 0;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float zp = round_dt<DT>(v[j] / md.Tr);
      keys[j] = f2key(zp);
      const int b = static_cast<int>(keys[j] >> BIN_SHIFT);
      const unsigned long long q = j < nv ? quant(wexp(zp, Mp)) : 0ull;
      tot += q;
      if (b > bhi) above += q;
      if (j < nv && b >= static_cast<int>(blo) && b <= bhi) cm |= 1u << j;
    }
    if (st.kind == KIND_HIST) {
      int total;
      const int cnt = __popc(cm);
      const int ex = block_excl_scan<int, 4>(cnt, s_scan, &total);
      int pos = ncand + ex;
#pragma unroll
      for (int j = 0; j < VEC; ++j)
        if (cm & (1u << j)) cand[pos++] = make_uint2(keys[j], static_cast<unsigned int>(i0 + j));
      ncand += total;
    }
  }
  tot = block_sum<unsigned long long, 4>(tot, s_u64);
  above = block_sum<unsigned long long, 4>(above, s_u64);
  if (tid == 0) {
    SliceMass m;
    m.above = above;
    m.total = tot;
    m.ncand = static_cast<unsigned int>(ncand);
    m.pad0 = 0;
    m.pad1 = 0;
    a.sm[r * a.S + s] = m;
  }
}

// ================================================================= k_select ==

// Candidate list of one row: per-slice regions concatenated in slice order.
struct CandView {
  const uint2* g;   // global base of the row's regions
  const uint2* l;   // LDS copy, or nullptr
  const int* off;   // [S+1] prefix of per-slice counts (LDS)
  int S, L;
  __device__ __forceinline__ uint2 get(int c) const {
    if (l) return l[c];
    int lo = 0, hi = S;  // slice s with off[s] <= c < off[s+1]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (off[mid] <= c)
        lo = mid;
      else
        hi = mid;
    }
    return g[static_cast<size_t>(lo) * L + (c - off[lo])];
  }
};

// Digit (descending) at which the running total crosses `target`, over a
// 256-bin histogram held in LDS; wave 0 only.  Returns the digit and, through
// *before, the sum of the digits above it.  `mode_count`: crossing is
// before < target <= before + h[d]; mass mode: first d with before + h[d] >=
// target (falls back to the lowest non-empty digit via cnt).
template <typename T>
__device__ __forceinline__ int find_digit(const T* h, const unsigned int* cnt, T target, T* before,
                                          bool* none) {
  const int lane = threadIdx.x & 63;
  T loc[4];
  T sum = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    loc[j] = h[255 - (4 * lane + j)];
    sum += loc[j];
  }
  T inc = wave_incl_scan(sum);
  T ex = inc - sum;
  int found = 256;
  T bef = 0;
  T run = ex;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (found == 256 && run + loc[j] >= target && loc[j] > 0) {
      found = 4 * lane + j;
      bef = run;
    }
    run += loc[j];
  }
  // lowest descending position with a hit
  int best = found;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) best = min(best, __shfl_xor(best, o, 64));
  T bsel = 0;
  const unsigned long long who = __ballot(found == best && best < 256);
  if (who) {
    const int src = __ffsll(static_cast<long long>(who)) - 1;
    bsel = __shfl(bef, src, 64);
  }
  if (best < 256) {
    *none = false;
    *before = bsel;
    return 255 - best;
  }
  // no crossing: lowest non-empty digit, everything above it counted
  int low = -1;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (cnt[255 - (4 * lane + j)]) low = max(low, 4 * lane + j);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) low = max(low, __shfl_xor(low, o, 64));
  T bsum = 0;
#pragma unroll
  for (int j = 0; j < 4; ++j)
    if (4 * lane + j < low) bsum += loc[j];
  bsum = wave_sum(bsum);
  *none = true;
  *before = bsum;
  return low < 0 ? 0 : 255 - low;
}

template <int DT>
__global__ __launch_bounds__(ROW_THREADS) void k_select(Args a) {
  __shared__ uint2 s_cand[CAND_LDS];
  __shared__ unsigned int s_hc[256];
  __shared__ unsigned long long s_hm[256];
  __shared__ int s_off[MAX_S + 1];
  __shared__ unsigned long long s_above[MAX_S];
  __shared__ unsigned long long s_total[MAX_S];
  __shared__ unsigned long long s_keep[MAX_S];
  __shared__ unsigned long long s_u64[ROW_WAVES + 1];
  __shared__ int s_int[ROW_WAVES + 1];
  __shared__ unsigned int s_sel[4];
  __shared__ unsigned long long s_selm[2];
  __shared__ int s_cut;

  const int r = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  RowState st = a.rs[r];
  if (st.kind == KIND_GREEDY) return;
  const Mode md = decode<DT>(a, r);
  const int S = a.S;

  if (tid < S) {
    const SliceMass m = a.sm[r * S + tid];
    s_above[tid] = m.above;
    s_total[tid] = m.total;
    s_keep[tid] = m.above;
    s_off[tid + 1] = static_cast<int>(m.ncand);
  }
  if (tid == 0) s_off[0] = 0;
  __syncthreads();
  if (tid == 0)
    for (int t = 0; t < S; ++t) s_off[t + 1] += s_off[t];
  __syncthreads();

  unsigned int vkey = 0;
  int idx_cut = INT_MAX;
  unsigned long long W = 0;

  if (st.kind == KIND_TEMP) {
    for (int t = 0; t < S; ++t) W += s_total[t];
    if (tid < S) s_keep[tid] = s_total[tid];
  } else {
    const int n = s_off[S];
    const uint2* g = a.cand + static_cast<size_t>(r) * S * a.L;
    const bool in_lds = n <= CAND_LDS;
    if (in_lds) {
      for (int t = 0; t < S; ++t) {
        const int o = s_off[t], cnt = s_off[t + 1] - o;
        for (int j = tid; j < cnt; j += ROW_THREADS) s_cand[o + j] = g[static_cast<size_t>(t) * a.L + j];
      }
    }
    __syncthreads();
    CandView cv;
    cv.g = g;
    cv.l = in_lds ? s_cand : nullptr;
    cv.off = s_off;
    cv.S = S;
    cv.L = a.L;

    unsigned long long mass_above = 0;
    for (int t = 0; t < S; ++t) mass_above += s_above[t];

    // (1) top-k: k_rel-th largest key among candidates (ties kept)
    unsigned int tau = 0;
    if (md.kk > 0) {
      unsigned int prefix = 0, mask = 0;
      unsigned int krel = static_cast<unsigned int>(md.kk) - st.cnt_above;
      for (int shift = 24; shift >= 0; shift -= 8) {
        for (int d = tid; d < 256; d += ROW_THREADS) s_hc[d] = 0u;
        __syncthreads();
        for (int c = tid; c < n; c += ROW_THREADS) {
          const unsigned int key = cv.get(c).x;
          if ((key & mask) == prefix) atomicAdd(&s_hc[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (wid == 0) {
          unsigned int bef;
          bool none;
          const int d = find_digit<unsigned int>(s_hc, s_hc, krel, &bef, &none);
          if (lane == 0) {
            s_sel[0] = static_cast<unsigned int>(d);
            s_sel[1] = bef;
          }
        }
        __syncthreads();
        prefix |= s_sel[0] << shift;
        mask |= 255u << shift;
        krel -= s_sel[1];
        __syncthreads();
      }
      tau = prefix;
    }

    // (2) mass of the top-k set: the candidates >= tau plus everything above R
    // (bins below R are below tau).  Without top-k it is the whole row.
    unsigned long long wk = 0;
    if (md.kk > 0) {
      for (int c = tid; c < n; c += ROW_THREADS) {
        const unsigned int key = cv.get(c).x;
        if (key >= tau) wk += quant(wexp(key2f(key), st.Mp));
      }
      wk = block_sum<unsigned long long, ROW_WAVES>(wk, s_u64) + mass_above;
    } else {
      for (int t = 0; t < S; ++t) wk += s_total[t];
    }

    if (!md.topp) {
      vkey = tau;
      idx_cut = INT_MAX;
      W = wk;
    } else {
      // (3) nucleus: smallest v with (mass strictly above v) < p * W_k
      const double x = static_cast<double>(md.pr) * static_cast<double>(wk);
      const unsigned long long PW = static_cast<unsigned long long>(ceil(x));
      unsigned long long P = mass_above;
      unsigned int prefix = 0, mask = 0;
      bool all_kept = false;
      unsigned int gcount = 0;
      for (int shift = 24; shift >= 0; shift -= 8) {
        for (int d = tid; d < 256; d += ROW_THREADS) {
          s_hc[d] = 0u;
          s_hm[d] = 0ull;
        }
        __syncthreads();
        for (int c = tid; c < n; c += ROW_THREADS) {
          const unsigned int key = cv.get(c).x;
          if (key >= tau && (key & mask) == prefix) {
            const unsigned int d = (key >> shift) & 255u;
            atomicAdd(&s_hc[d], 1u);
            const unsigned long long q = quant(wexp(key2f(key), st.Mp));
            if (q) atomicAdd(&s_hm[d], q);
          }
        }
        __syncthreads();
        if (wid == 0) {
          unsigned long long bef;
          bool none;
          // all_kept rounds keep picking the lowest non-empty digit
          const unsigned long long tgt = all_kept ? ~0ull : (PW > P ? PW - P : 0ull);
          const int d = find_digit<unsigned long long>(s_hm, s_hc, tgt, &bef, &none);
          if (lane == 0) {
            s_sel[0] = static_cast<unsigned int>(d);
            s_sel[1] = none ? 1u : 0u;
            s_sel[2] = s_hc[d];
            s_selm[0] = bef;
          }
        }
        __syncthreads();
        prefix |= s_sel[0] << shift;
        mask |= 255u << shift;
        P += s_selm[0];
        all_kept = all_kept || (s_sel[1] != 0u);
        gcount = s_sel[2];
        __syncthreads();
      }
      vkey = prefix;
      const unsigned long long wstar = quant(wexp(key2f(vkey), st.Mp));
      unsigned long long t = gcount;
      if (!all_kept && wstar > 0) {
        const unsigned long long need = (PW - P + wstar - 1) / wstar;
        t = need < t ? need : t;
      }
      W = P + t * wstar;
      // (4) index cut: the t-th candidate (buffer = index order) with key == v*
      if (t >= gcount) {
        idx_cut = INT_MAX;
      } else {
        const int per = (n + ROW_THREADS - 1) / ROW_THREADS;
        const int c0 = tid * per, c1 = min(n, c0 + per);
        int cnt = 0;
        for (int c = c0; c < c1; ++c) cnt += cv.get(c).x == vkey ? 1 : 0;
        int tot;
        const int ex = block_excl_scan<int, ROW_WAVES>(cnt, s_int, &tot);
        if (tid == 0) s_cut = INT_MAX;
        __syncthreads();
        const int want = static_cast<int>(t);  // 1-based rank
        if (ex < want && ex + cnt >= want) {
          int seen = ex;
          for (int c = c0; c < c1; ++c) {
            const uint2 e = cv.get(c);
            if (e.x == vkey && ++seen == want) {
              s_cut = static_cast<int>(e.y);
              break;
            }
          }
        }
        __syncthreads();
        idx_cut = s_cut;
      }
    }
    // (5) kept mass per slice
    for (int c = tid; c < n; c += ROW_THREADS) {
      const uint2 e = cv.get(c);
      const int idx = static_cast<int>(e.y);
      if (e.x > vkey || (e.x == vkey && idx <= idx_cut)) {
        const unsigned long long q = quant(wexp(key2f(e.x), st.Mp));
        if (q) atomicAdd(&s_keep[idx / a.L], q);
      }
    }
    __syncthreads();
  }

  if (tid == 0) {
    unsigned long long tot = 0;
    for (int t = 0; t < S; ++t) tot += s_keep[t];
    W = tot;
    const double x = static_cast<double>(md.u) * static_cast<double>(W);
    unsigned long long tg = static_cast<unsigned long long>(x);
    if (W == 0)
      tg = 0;
    else if (tg >= W)
      tg = W - 1;
    unsigned long long cum = 0;
    int sst = S - 1;
    for (int t = 0; t < S; ++t) {
      if (cum + s_keep[t] > tg) {
        sst = t;
        break;
      }
      cum += s_keep[t];
    }
    a.rs[r].vkey = vkey;
    a.rs[r].idx_cut = idx_cut;
    a.rs[r].s_star = sst;
    a.rs[r].target_rem = tg - cum;
  }
}

// =================================================================== k_draw ==

template <int DT, bool VECOK>
__global__ __launch_bounds__(ROW_THREADS) void k_draw(Args a) {
  __shared__ unsigned long long s_u64[ROW_WAVES + 1];
  __shared__ int s_found;

  const int r = blockIdx.x;
  const int tid = threadIdx.x;
  const RowState st = a.rs[r];
  if (st.kind == KIND_GREEDY) return;
  const Mode md = decode<DT>(a, r);
  const void* row = row_ptr<DT>(a, r);
  const int beg = st.s_star * a.L;
  const int end = min(a.V, beg + a.L);
  unsigned long long rem = st.target_rem;
  if (tid == 0) s_found = -1;
  __syncthreads();
  for (int base = beg; base < end; base += ROW_THREADS * VEC) {
    const int i0 = base + tid * VEC;
    float v[VEC];
    int nv;
    load8<DT, VECOK>(row, i0, end, v, nv);
    unsigned long long q[VEC];
    unsigned long long sum = 0;
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float zp = round_dt<DT>(v[j] / md.Tr);
      const unsigned int key = f2key(zp);
      const bool kept = j < nv && (key > st.vkey || (key == st.vkey && i0 + j <= st.idx_cut));
      q[j] = kept ? quant(wexp(zp, st.Mp)) : 0ull;
      sum += q[j];
    }
    unsigned long long total;
    const unsigned long long ex = block_excl_scan<unsigned long long, ROW_WAVES>(sum, s_u64, &total);
    if (ex <= rem && rem < ex + sum) {
      unsigned long long c = ex;
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        c += q[j];
        if (c > rem) {
          s_found = i0 + j;
          break;
        }
      }
    }
    __syncthreads();
    if (s_found >= 0) break;
    rem -= total;
  }
  if (tid == 0) {
    int id = s_found;
    if (id < 0) id = beg;  // unreachable: the slice's kept mass exceeds rem
    a.out_ids[r] = id;
    if (a.out_lp) {
      if (md.want_lp) {
        const float z = ld1<DT>(row, id);
        a.out_lp[r] = static_cast<float>(static_cast<double>(z) - st.lse);
      } else {
        a.out_lp[r] = NAN;
      }
    }
  }
}

// ================================================================ host side ==

struct Layout {
  int S, L;
  size_t off_rs, off_rec, off_top, off_hcnt, off_hmass, off_sm, off_cand, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

Layout make_layout(int B, int V, int K_max) {
  Layout l;
  int S0 = (TARGET_BLOCKS + B - 1) / (B > 0 ? B : 1);
  S0 = S0 < 1 ? 1 : (S0 > MAX_S ? MAX_S : S0);
  int L = (V + S0 - 1) / S0;
  L = (L + ITER_ELEMS - 1) / ITER_ELEMS * ITER_ELEMS;
  l.S = (V + L - 1) / L;
  l.L = L;
  const size_t BS = static_cast<size_t>(B) * l.S;
  size_t o = 0;
  l.off_rs = o;
  o = align256(o + sizeof(RowState) * B);
  l.off_rec = o;
  o = align256(o + sizeof(SliceRec) * BS);
  l.off_top = o;
  o = align256(o + sizeof(TopEnt) * BS * (K_max > 0 ? K_max : 1));
  l.off_hcnt = o;
  o = align256(o + sizeof(unsigned int) * BS * NB);
  l.off_hmass = o;
  o = align256(o + sizeof(unsigned long long) * BS * NB);
  l.off_sm = o;
  o = align256(o + sizeof(SliceMass) * BS);
  l.off_cand = o;
  o = align256(o + sizeof(uint2) * BS * l.L);
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

constexpr int NUM_STAGES = 5;

// ev (optional): NUM_STAGES + 1 events recorded around the kernels.
template <int DT, bool VECOK>
hipError_t launch_all(const Args& a, hipStream_t st, hipEvent_t* ev) {
  const dim3 slices(a.S, a.B);
  auto mark = [&](int i) {
    if (ev) (void)hipEventRecord(ev[i], st);
  };
  mark(0);
  hipLaunchKernelGGL((k_scan<DT, VECOK>), slices, dim3(SLICE_THREADS), 0, st, a);
  mark(1);
  hipLaunchKernelGGL((k_plan<DT>), dim3(a.B), dim3(ROW_THREADS), 0, st, a);
  mark(2);
  if (a.T) {
    hipLaunchKernelGGL((k_extract<DT, VECOK>), slices, dim3(SLICE_THREADS), 0, st, a);
    mark(3);
    hipLaunchKernelGGL((k_select<DT>), dim3(a.B), dim3(ROW_THREADS), 0, st, a);
    mark(4);
    hipLaunchKernelGGL((k_draw<DT, VECOK>), dim3(a.B), dim3(ROW_THREADS), 0, st, a);
    mark(5);
  } else {
    mark(3);
    mark(4);
    mark(5);
  }
  return hipGetLastError();
}

template <int DT>
hipError_t dispatch_vec(const Args& a, bool vecok, hipStream_t st, hipEvent_t* ev) {
  return vecok ? launch_all<DT, true>(a, st, ev) : launch_all<DT, false>(a, st, ev);
}

}  // namespace

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
    *bytes = make_layout(B, V, K_max).total;
    return MLXF_OK;
  } catch (...) {
    set_err(err, "mlxf: unexpected exception");
    return MLXF_EINVAL;
  }
}

}  // extern "C"

namespace {

int run_sample(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
               const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
               const int32_t* d_top_logprobs, const float* d_uniforms, int32_t* d_out_ids,
               float* d_out_logprobs, int32_t* d_out_top_ids, float* d_out_top_logprobs,
               int K_max, void* d_workspace, size_t workspace_bytes, void* stream, char** err,
               hipEvent_t* ev) {
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
    const Layout l = make_layout(B, V, K_max);
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
    Args a;
    a.logits = d_logits;
    a.row_stride = row_stride;
    a.B = B;
    a.V = V;
    a.K_max = K_max;
    a.S = l.S;
    a.L = l.L;
    a.T = d_temperature;
    a.k = d_top_k;
    a.p = d_top_p;
    a.tlp = d_top_logprobs;
    a.u = d_uniforms;
    a.out_ids = d_out_ids;
    a.out_lp = d_out_logprobs;
    a.out_top_ids = d_out_top_ids;
    a.out_top_lp = d_out_top_logprobs;
    a.rs = reinterpret_cast<RowState*>(ws + l.off_rs);
    a.rec = reinterpret_cast<SliceRec*>(ws + l.off_rec);
    a.top = reinterpret_cast<TopEnt*>(ws + l.off_top);
    a.hcnt = reinterpret_cast<unsigned int*>(ws + l.off_hcnt);
    a.hmass = reinterpret_cast<unsigned long long*>(ws + l.off_hmass);
    a.sm = reinterpret_cast<SliceMass*>(ws + l.off_sm);
    a.cand = reinterpret_cast<uint2*>(ws + l.off_cand);
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e;
    if (dtype == MLXF_DTYPE_F32)
      e = dispatch_vec<MLXF_DTYPE_F32>(a, vecok, st, ev);
    else if (dtype == MLXF_DTYPE_BF16)
      e = dispatch_vec<MLXF_DTYPE_BF16>(a, vecok, st, ev);
    else
      e = dispatch_vec<MLXF_DTYPE_F16>(a, vecok, st, ev);
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

}  // namespace

extern "C" {

int mlxf_sample(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                const int32_t* d_top_logprobs, const float* d_uniforms, int32_t* d_out_ids,
                float* d_out_logprobs, int32_t* d_out_top_ids, float* d_out_top_logprobs,
                int K_max, void* d_workspace, size_t workspace_bytes, void* stream, char** err) {
  return run_sample(d_logits, dtype, B, V, row_stride, d_temperature, d_top_k, d_top_p,
                    d_top_logprobs, d_uniforms, d_out_ids, d_out_logprobs, d_out_top_ids,
                    d_out_top_logprobs, K_max, d_workspace, workspace_bytes, stream, err, nullptr);
}

int mlxf_sample_profiled(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                         const float* d_temperature, const int32_t* d_top_k,
                         const float* d_top_p, const int32_t* d_top_logprobs,
                         const float* d_uniforms, int32_t* d_out_ids, float* d_out_logprobs,
                         int32_t* d_out_top_ids, float* d_out_top_logprobs, int K_max,
                         void* d_workspace, size_t workspace_bytes, void* stream,
                         float* stage_ms, char** err) {
  if (!stage_ms) {
    set_err(err, "mlxf: stage_ms must not be NULL");
    return MLXF_EINVAL;
  }
  hipEvent_t ev[NUM_STAGES + 1] = {};
  for (int i = 0; i <= NUM_STAGES; ++i) {
    if (hipEventCreate(&ev[i]) != hipSuccess) {
      for (int j = 0; j < i; ++j) (void)hipEventDestroy(ev[j]);
      set_err(err, "mlxf: hipEventCreate failed");
      return MLXF_EHIP;
    }
  }
  int rc = run_sample(d_logits, dtype, B, V, row_stride, d_temperature, d_top_k, d_top_p,
                      d_top_logprobs, d_uniforms, d_out_ids, d_out_logprobs, d_out_top_ids,
                      d_out_top_logprobs, K_max, d_workspace, workspace_bytes, stream, err, ev);
  if (rc == MLXF_OK && B > 0) {
    if (hipEventSynchronize(ev[NUM_STAGES]) != hipSuccess) {
      set_err(err, "mlxf: hipEventSynchronize failed");
      rc = MLXF_EHIP;
    } else {
      for (int i = 0; i < NUM_STAGES; ++i) {
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, ev[i], ev[i + 1]);
        stage_ms[i] = ms;
      }
    }
  }
  for (int i = 0; i <= NUM_STAGES; ++i) (void)hipEventDestroy(ev[i]);
  return rc;
}

int mlxf_greedy(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                int32_t* d_out_ids, void* d_workspace, size_t workspace_bytes, void* stream,
                char** err) {
  return mlxf_sample(d_logits, dtype, B, V, row_stride, nullptr, nullptr, nullptr, nullptr,
                     nullptr, d_out_ids, nullptr, nullptr, nullptr, 0, d_workspace,
                     workspace_bytes, stream, err);
}

}  // extern "C"
