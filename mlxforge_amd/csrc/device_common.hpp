// device_common.hpp -- device helpers of the gfx950 sampler: monotone float
// keys, dtype rounding, raw vector loads, the weight function, lane exchanges,
// DPP wave / block scans and the best-64 list sort / merge.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <climits>

#include "mlxf_sampler.h"

namespace mlxf {

constexpr int THREADS = 256;  // one workgroup per row slice; 4 waves, one per SIMD
constexpr int WAVES = THREADS / 64;
constexpr int VEC = 8;                  // elements per 16-byte (bf16/f16) or 32-byte (f32) load
constexpr int CHUNK = THREADS * VEC;    // elements one load instruction covers across the block
constexpr int MAX_S = 64;               // slices per row (<= 64: one wave combines them)
constexpr float LOG2E = 1.4426950408889634f;
constexpr unsigned int KEY_NEG_INF = 0x007fffffu;  // key of -inf; smaller keys are NaNs
constexpr unsigned int KEY_POS_INF = 0xff800000u;

// Monotone unsigned key of a float: a < b  <=>  key(a) < key(b) (no NaNs).
__device__ __forceinline__ unsigned int f2key(float f) {
  const unsigned int u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key2f(unsigned int k) {
  const unsigned int u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
  return __uint_as_float(u);
}

// Round-to-nearest-even into the logits dtype (the temperature division of
// src/sample/sampler.cpp:158 is carried out in the logits dtype).
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

// z' = round_dtype(z / T), IEEE division.  Monotone non-decreasing in z.
template <int DT>
__device__ __forceinline__ float fz(float z, float Tr) {
  return round_dt<DT>(z / Tr);
}

// Smallest key k (over non-NaN floats) with fz(key2f(k)) >= y.
template <int DT>
__device__ __forceinline__ unsigned int gkey(float y, float Tr) {
  unsigned int lo = KEY_NEG_INF, hi = KEY_POS_INF;
  if (!(fz<DT>(INFINITY, Tr) >= y)) return KEY_POS_INF;
  while (lo < hi) {
    const unsigned int mid = lo + ((hi - lo) >> 1);
    if (fz<DT>(key2f(mid), Tr) >= y)
      hi = mid;
    else
      lo = mid + 1;
  }
  return lo;
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

// Raw storage of 8 consecutive elements: two 16-byte words for fp32, one for
// the 16-bit types.  Loading raw and decoding later keeps several slices'
// loads in flight in few registers.
template <int DT>
struct Raw8 {
  static constexpr int NQ = DT == MLXF_DTYPE_F32 ? 2 : 1;
  uint4 q[NQ];
};

template <int DT>
__device__ __forceinline__ unsigned int neg_inf_bits() {
  return DT == MLXF_DTYPE_F32 ? 0xff800000u : (DT == MLXF_DTYPE_BF16 ? 0xff80u : 0xfc00u);
}

template <int DT>
__device__ __forceinline__ unsigned int ld_bits(const void* row, int i) {
  if constexpr (DT == MLXF_DTYPE_F32)
    return static_cast<const unsigned int*>(row)[i];
  else
    return static_cast<const unsigned short*>(row)[i];
}

// 8 consecutive elements from i0 (i0 % 8 == 0); entries at or past `end` read
// as -inf.
template <int DT, bool VECOK>
__device__ __forceinline__ void load_raw(const void* row, int i0, int end, Raw8<DT>& r) {
  const int nv = end - i0;
  if (VECOK && nv >= VEC) {
    const uint4* p = reinterpret_cast<const uint4*>(static_cast<const char*>(row) +
                                                    static_cast<size_t>(i0) * elem_size<DT>());
#pragma unroll
    for (int q = 0; q < Raw8<DT>::NQ; ++q) r.q[q] = p[q];
  } else {
    unsigned int b[VEC];
#pragma unroll
    for (int j = 0; j < VEC; ++j) b[j] = j < nv ? ld_bits<DT>(row, i0 + j) : neg_inf_bits<DT>();
    if constexpr (DT == MLXF_DTYPE_F32) {
      r.q[0] = make_uint4(b[0], b[1], b[2], b[3]);
      r.q[1] = make_uint4(b[4], b[5], b[6], b[7]);
    } else {
      r.q[0] = make_uint4(b[0] | (b[1] << 16), b[2] | (b[3] << 16), b[4] | (b[5] << 16),
                          b[6] | (b[7] << 16));
    }
  }
}

// Raw -> fp32 values, NaN kept.
template <int DT>
__device__ __forceinline__ void decode8_nan(const Raw8<DT>& r, float* v) {
  if constexpr (DT == MLXF_DTYPE_F32) {
    const unsigned int w[8] = {r.q[0].x, r.q[0].y, r.q[0].z, r.q[0].w,
                               r.q[1].x, r.q[1].y, r.q[1].z, r.q[1].w};
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __uint_as_float(w[j]);
  } else {
    const unsigned int w[4] = {r.q[0].x, r.q[0].y, r.q[0].z, r.q[0].w};
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
}

// Raw -> fp32 values; NaN reads as -inf.
template <int DT>
__device__ __forceinline__ void decode8(const Raw8<DT>& r, float* v) {
  decode8_nan<DT>(r, v);
#pragma unroll
  for (int j = 0; j < VEC; ++j) v[j] = v[j] != v[j] ? -INFINITY : v[j];
}

// Three-operand maximum / minimum / minimum of magnitudes.  The inputs must not
// be NaN (callers clear NaNs first): then the instruction is the exact
// maximum or minimum, and asm keeps the compiler from adding the quieting
// instructions it puts before a max of values it cannot prove NaN-free.
__device__ __forceinline__ float vmax3(float a, float b, float c) {
  float d;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}
__device__ __forceinline__ float vmin3(float a, float b, float c) {
  float d;
  asm("v_min3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}
__device__ __forceinline__ float vmin3_abs(float a, float b, float c) {  // min(a, |b|, |c|)
  float d;
  asm("v_min3_f32 %0, %1, |%2|, |%3|" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}

// n values, NaN read as -inf.  A NaN is found from two maxima of the bit
// patterns (unsigned: a negative NaN lies above -inf; signed: a positive NaN
// above +inf), and only a wave holding one rewrites its values.
template <int N>
__device__ __forceinline__ void clear_nans(float (&v)[N]) {
  unsigned int hu = 0u;
  int hs = INT_MIN;
#pragma unroll
  for (int e = 0; e < N; ++e) {
    hu = max(hu, __float_as_uint(v[e]));
    hs = max(hs, static_cast<int>(__float_as_uint(v[e])));
  }
  if (__builtin_amdgcn_ballot_w64(hu > 0xff800000u || hs > 0x7f800000)) {
#pragma unroll
    for (int e = 0; e < N; ++e) v[e] = v[e] != v[e] ? -INFINITY : v[e];
  }
}

template <int DT, bool VECOK>
__device__ __forceinline__ void load8(const void* row, int i0, int end, float* v) {
  Raw8<DT> r;
  load_raw<DT, VECOK>(row, i0, end, r);
  decode8<DT>(r, v);
}
template <int DT, bool VECOK>
__device__ __forceinline__ void load8_nan(const void* row, int i0, int end, float* v) {
  Raw8<DT> r;
  load_raw<DT, VECOK>(row, i0, end, r);
  decode8_nan<DT>(r, v);
}

// exp(x - m) with exp(m - m) = 1 also for infinite m.
__device__ __forceinline__ float wexp(float x, float m) {
  const float e = __builtin_amdgcn_exp2f((x - m) * LOG2E);
  return x == m ? 1.0f : e;
}
__device__ __forceinline__ double wexp_d(float x, float m) {
  return x == m ? 1.0 : exp(static_cast<double>(x) - static_cast<double>(m));
}

__device__ __forceinline__ unsigned long long pack2(unsigned int lo, unsigned int hi) {
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

// (av, ai) before (bv, bi) in (value desc, index asc) order.  Bitwise, not
// short-circuit: the short-circuit form compiles to exec-mask branches.
__device__ __forceinline__ bool better(float av, int ai, float bv, int bi) {
  return (av > bv) | ((av == bv) & (ai < bi));
}

// ---- cross-lane exchange on the VALU (DPP and gfx950 permlane swaps; no
// LDS round trip as ds_bpermute would take).  xshf<M>(x) is lane (lane ^ M)'s
// value.  Call only with the whole wave active.
template <int M>
__device__ __forceinline__ int xshf_i(int v) {
  const int lane = threadIdx.x & 63;
  if constexpr (M == 1) {
    return __builtin_amdgcn_mov_dpp(v, 0xb1, 0xf, 0xf, false);  // quad_perm [1,0,3,2]
  } else if constexpr (M == 2) {
    return __builtin_amdgcn_mov_dpp(v, 0x4e, 0xf, 0xf, false);  // quad_perm [2,3,0,1]
  } else if constexpr (M == 4) {
    const int dn = __builtin_amdgcn_mov_dpp(v, 0x124, 0xf, 0xf, false);  // row_ror:4  (i - 4)
    const int up = __builtin_amdgcn_mov_dpp(v, 0x12c, 0xf, 0xf, false);  // row_ror:12 (i + 4)
    return (lane & 4) ? dn : up;
  } else if constexpr (M == 8) {
    return __builtin_amdgcn_mov_dpp(v, 0x128, 0xf, 0xf, false);  // row_ror:8
  } else if constexpr (M == 15) {
    return __builtin_amdgcn_mov_dpp(v, 0x140, 0xf, 0xf, false);  // row_mirror
  } else if constexpr (M == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
    return static_cast<int>((lane & 16) ? r[0] : r[1]);
  } else {
    static_assert(M == 32, "xor distance");
    const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
    return static_cast<int>((lane & 32) ? r[0] : r[1]);
  }
}
template <int M>
__device__ __forceinline__ int xshf(int v) { return xshf_i<M>(v); }
template <int M>
__device__ __forceinline__ unsigned int xshf(unsigned int v) {
  return static_cast<unsigned int>(xshf_i<M>(static_cast<int>(v)));
}
template <int M>
__device__ __forceinline__ float xshf(float v) { return __int_as_float(xshf_i<M>(__float_as_int(v))); }
template <int M>
__device__ __forceinline__ unsigned long long xshf(unsigned long long v) {
  const unsigned int lo = xshf<M>(static_cast<unsigned int>(v));
  const unsigned int hi = xshf<M>(static_cast<unsigned int>(v >> 32));
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}
template <int M>
__device__ __forceinline__ long long xshf(long long v) {
  return static_cast<long long>(xshf<M>(static_cast<unsigned long long>(v)));
}
template <int M>
__device__ __forceinline__ double xshf(double v) { return __longlong_as_double(xshf<M>(__double_as_longlong(v))); }

// Value of a wave-uniform lane `src` (v_readlane: scalar, no LDS).
__device__ __forceinline__ int rdl(int v, int src) { return __builtin_amdgcn_readlane(v, src); }
__device__ __forceinline__ unsigned int rdl(unsigned int v, int src) {
  return static_cast<unsigned int>(__builtin_amdgcn_readlane(static_cast<int>(v), src));
}
__device__ __forceinline__ float rdl(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}
__device__ __forceinline__ double rdl(double v, int src) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane(static_cast<int>(b), src);
  const int hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), src);
  return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
}
__device__ __forceinline__ unsigned long long rdl(unsigned long long v, int src) {
  const unsigned int lo = rdl(static_cast<unsigned int>(v), src);
  const unsigned int hi = rdl(static_cast<unsigned int>(v >> 32), src);
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

// Butterfly sum: every lane ends with the same value (each step adds the same
// two operands in either order).
template <typename T>
__device__ __forceinline__ T wave_sum(T x) {
  x += xshf<32>(x);
  x += xshf<16>(x);
  x += xshf<8>(x);
  x += xshf<4>(x);
  x += xshf<2>(x);
  x += xshf<1>(x);
  return x;
}
template <typename T>
__device__ __forceinline__ T wave_max(T x) {
  x = max(x, xshf<32>(x));
  x = max(x, xshf<16>(x));
  x = max(x, xshf<8>(x));
  x = max(x, xshf<4>(x));
  x = max(x, xshf<2>(x));
  x = max(x, xshf<1>(x));
  return x;
}
template <typename T>
__device__ __forceinline__ T wave_min(T x) {
  x = min(x, xshf<32>(x));
  x = min(x, xshf<16>(x));
  x = min(x, xshf<8>(x));
  x = min(x, xshf<4>(x));
  x = min(x, xshf<2>(x));
  x = min(x, xshf<1>(x));
  return x;
}

// Inclusive scan of an int over the wave on the VALU: shifts within each row
// of 16 lanes, then the rows' last lanes broadcast forward (row_bcast:15 into
// rows 1 and 3, row_bcast:31 into rows 2 and 3).  Whole wave active.
__device__ __forceinline__ int wave_incl_scan_dpp(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);  // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}

// Lane move of a double by DPP control CTRL (row mask RM; lanes without a
// source, or outside RM, read 0.0).
template <int CTRL, int RM, bool BC>
__device__ __forceinline__ double dpp_d(double x) {
  const long long b = __double_as_longlong(x);
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(b), CTRL, RM, 0xf, BC);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(b >> 32), CTRL, RM, 0xf, BC);
  return __longlong_as_double((static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
}

// Inclusive scan of a double over the wave, same lane pattern as
// wave_incl_scan_dpp.  Exact for integer values whose sums stay below 2^53.
__device__ __forceinline__ double wave_incl_scan_dpp(double x) {
  x += dpp_d<0x111, 0xf, true>(x);
  x += dpp_d<0x112, 0xf, true>(x);
  x += dpp_d<0x114, 0xf, true>(x);
  x += dpp_d<0x118, 0xf, true>(x);
  x += dpp_d<0x142, 0xa, false>(x);
  x += dpp_d<0x143, 0xc, false>(x);
  return x;
}

// Lane move of a 64-bit integer by DPP control CTRL (as dpp_d).
template <int CTRL, int RM, bool BC>
__device__ __forceinline__ unsigned long long dpp_u64(unsigned long long x) {
  const int lo = __builtin_amdgcn_update_dpp(0, static_cast<int>(x), CTRL, RM, 0xf, BC);
  const int hi = __builtin_amdgcn_update_dpp(0, static_cast<int>(x >> 32), CTRL, RM, 0xf, BC);
  return (static_cast<unsigned long long>(static_cast<unsigned int>(hi)) << 32) | static_cast<unsigned int>(lo);
}

// Inclusive scan of a 64-bit integer over the wave (lane pattern of
// wave_incl_scan_dpp).
__device__ __forceinline__ unsigned long long wave_incl_scan_dpp(unsigned long long x) {
  x += dpp_u64<0x111, 0xf, true>(x);
  x += dpp_u64<0x112, 0xf, true>(x);
  x += dpp_u64<0x114, 0xf, true>(x);
  x += dpp_u64<0x118, 0xf, true>(x);
  x += dpp_u64<0x142, 0xa, false>(x);
  x += dpp_u64<0x143, 0xc, false>(x);
  return x;
}

// Inclusive scan within each row of 16 lanes (row_shr steps only; lanes
// without a source add 0).  Whole wave active.
__device__ __forceinline__ int row_incl_scan16(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);  // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);  // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);  // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);  // row_shr:8
  return x;
}
__device__ __forceinline__ unsigned long long row_incl_scan16(unsigned long long x) {
  x += dpp_u64<0x111, 0xf, true>(x);
  x += dpp_u64<0x112, 0xf, true>(x);
  x += dpp_u64<0x114, 0xf, true>(x);
  x += dpp_u64<0x118, 0xf, true>(x);
  return x;
}

// Butterfly sum / max / min within each row of 16 lanes: every lane of a row
// ends with its row's result.  Whole wave active.
template <typename T>
__device__ __forceinline__ T row_sum16(T x) {
  x += xshf<8>(x);
  x += xshf<4>(x);
  x += xshf<2>(x);
  x += xshf<1>(x);
  return x;
}
template <typename T>
__device__ __forceinline__ T row_max16(T x) {
  x = max(x, xshf<8>(x));
  x = max(x, xshf<4>(x));
  x = max(x, xshf<2>(x));
  x = max(x, xshf<1>(x));
  return x;
}
template <typename T>
__device__ __forceinline__ T row_min16(T x) {
  x = min(x, xshf<8>(x));
  x = min(x, xshf<4>(x));
  x = min(x, xshf<2>(x));
  x = min(x, xshf<1>(x));
  return x;
}

// Exclusive block scan of an integer (int or 64-bit) for an lds array that no
// thread of the block has read since the last barrier: one barrier; *total is
// the block sum.  lds: WAVES entries.
template <typename T>
__device__ __forceinline__ T block_excl_scan_dpp(T x, T* lds, T* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const T inc = wave_incl_scan_dpp(x);
  if (lane == 63) lds[wid] = inc;
  __syncthreads();
  T off = 0, tot = 0;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    const T t = lds[w];
    off += w < wid ? t : T(0);
    tot += t;
  }
  *total = tot;
  return inc - x + off;
}

// Block sum in a fixed order (deterministic for floating T).  lds: WAVES entries.
template <typename T>
__device__ __forceinline__ T block_sum(T x, T* lds) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  x = wave_sum(x);
  __syncthreads();  // lds may still be read by a previous call
  if (lane == 0) lds[wid] = x;
  __syncthreads();
  T t = lds[0];
#pragma unroll
  for (int w = 1; w < WAVES; ++w) t += lds[w];
  return t;
}

// One compare-exchange stage at xor distance J: in `asc` runs the better
// entry moves to the lower lane.
template <int J>
__device__ __forceinline__ void cx(float& v, int& i, bool asc) {
  const int lane = threadIdx.x & 63;
  const float ov = xshf<J>(v);
  const int oi = xshf<J>(i);
  const bool first = (lane & J) == 0;
  const bool ob = better(ov, oi, v, i);
  if ((first == asc) ? ob : !ob) {
    v = ov;
    i = oi;
  }
}
template <int K>
__device__ __forceinline__ void bitonic_stage(float& v, int& i) {
  const bool asc = ((threadIdx.x & 63) & K) == 0;
  if constexpr (K >= 64) cx<32>(v, i, asc);
  if constexpr (K >= 32) cx<16>(v, i, asc);
  if constexpr (K >= 16) cx<8>(v, i, asc);
  if constexpr (K >= 8) cx<4>(v, i, asc);
  if constexpr (K >= 4) cx<2>(v, i, asc);
  cx<1>(v, i, asc);
}

// Bitonic sort of one entry per lane, best (v desc, i asc) in lane 0.
// Bitonic sort of (index, weight) pairs by ascending index (no equal indices
// but INT_MAX, whose weight is 0).
template <int J>
__device__ __forceinline__ void cx_idx(int& i, double& w, bool asc) {
  const int lane = threadIdx.x & 63;
  const int oi = xshf<J>(i);
  const double ow = xshf<J>(w);
  const bool first = (lane & J) == 0;
  const bool ob = oi < i;
  if ((first == asc) ? ob : !ob) {
    i = oi;
    w = ow;
  }
}
template <int K>
__device__ __forceinline__ void bitonic_stage_idx(int& i, double& w) {
  const bool asc = ((threadIdx.x & 63) & K) == 0;
  if constexpr (K >= 64) cx_idx<32>(i, w, asc);
  if constexpr (K >= 32) cx_idx<16>(i, w, asc);
  if constexpr (K >= 16) cx_idx<8>(i, w, asc);
  if constexpr (K >= 8) cx_idx<4>(i, w, asc);
  if constexpr (K >= 4) cx_idx<2>(i, w, asc);
  cx_idx<1>(i, w, asc);
}
__device__ __forceinline__ void wave_sort_idx(int& i, double& w) {
  bitonic_stage_idx<2>(i, w);
  bitonic_stage_idx<4>(i, w);
  bitonic_stage_idx<8>(i, w);
  bitonic_stage_idx<16>(i, w);
  bitonic_stage_idx<32>(i, w);
  bitonic_stage_idx<64>(i, w);
}

__device__ __forceinline__ void wave_sort(float& v, int& i) {
  bitonic_stage<2>(v, i);
  bitonic_stage<4>(v, i);
  bitonic_stage<8>(v, i);
  bitonic_stage<16>(v, i);
  bitonic_stage<32>(v, i);
  bitonic_stage<64>(v, i);
}

// Merge the sorted lane list (lv, li) with another sorted list (nv, ni),
// keeping the best 64: reverse the incoming list (lane ^ 63), keep the better
// of each pair, then one bitonic half-cleaning pass.
__device__ __forceinline__ void wave_list_merge(float& lv, int& li, float nv, int ni) {
  const float rv = xshf<32>(xshf<16>(xshf<15>(nv)));
  const int ri = xshf<32>(xshf<16>(xshf<15>(ni)));
  if (better(rv, ri, lv, li)) {
    lv = rv;
    li = ri;
  }
  cx<32>(lv, li, true);
  cx<16>(lv, li, true);
  cx<8>(lv, li, true);
  cx<4>(lv, li, true);
  cx<2>(lv, li, true);
  cx<1>(lv, li, true);
}

// Unsigned keys, one per lane, sorted descending across the wave (largest in
// lane 0); the same bitonic network on bare keys.
template <int J>
__device__ __forceinline__ void cxk(unsigned int& k, bool asc) {
  const unsigned int o = xshf<J>(k);
  const bool first = ((threadIdx.x & 63) & J) == 0;
  k = (first == asc) ? max(k, o) : min(k, o);
}
template <int K>
__device__ __forceinline__ void bitonic_stage_k(unsigned int& k) {
  const bool asc = ((threadIdx.x & 63) & K) == 0;
  if constexpr (K >= 64) cxk<32>(k, asc);
  if constexpr (K >= 32) cxk<16>(k, asc);
  if constexpr (K >= 16) cxk<8>(k, asc);
  if constexpr (K >= 8) cxk<4>(k, asc);
  if constexpr (K >= 4) cxk<2>(k, asc);
  cxk<1>(k, asc);
}
__device__ __forceinline__ void wave_sort_keys(unsigned int& k) {
  bitonic_stage_k<2>(k);
  bitonic_stage_k<4>(k);
  bitonic_stage_k<8>(k);
  bitonic_stage_k<16>(k);
  bitonic_stage_k<32>(k);
  bitonic_stage_k<64>(k);
}
// The 64 largest of two descending lane lists, descending (the incoming list
// reversed, the larger of each pair kept, one half-cleaning pass).
__device__ __forceinline__ void wave_merge_keys(unsigned int& l, unsigned int n) {
  l = max(l, xshf<32>(xshf<16>(xshf<15>(n))));
  cxk<32>(l, true);
  cxk<16>(l, true);
  cxk<8>(l, true);
  cxk<4>(l, true);
  cxk<2>(l, true);
  cxk<1>(l, true);
}

// Best (v desc, i asc) over the wave, in every lane.
__device__ __forceinline__ void wave_best(float& v, int& i) {
#define MLXF_BEST_STEP(M)                  \
  {                                        \
    const float ov = xshf<M>(v);           \
    const int oi = xshf<M>(i);             \
    if (better(ov, oi, v, i)) {            \
      v = ov;                              \
      i = oi;                              \
    }                                      \
  }
  MLXF_BEST_STEP(32)
  MLXF_BEST_STEP(16)
  MLXF_BEST_STEP(8)
  MLXF_BEST_STEP(4)
  MLXF_BEST_STEP(2)
  MLXF_BEST_STEP(1)
#undef MLXF_BEST_STEP
}

struct TopEnt {
  float v;
  int i;
};

// Waves [0, nw) each hold a sorted list (lv, li); on return wave 0 holds the
// best 64 of their union.  Pairwise rounds through `lists` (WAVES * 64 LDS
// entries).  Whole workgroup, nw uniform; ends with a barrier.
__device__ __forceinline__ void tree_merge(float& lv, int& li, TopEnt* lists, int nw) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  for (int n = nw; n > 1;) {
    const int h = (n + 1) >> 1;
    if (wid >= h && wid < n) {
      lists[wid * 64 + lane].v = lv;
      lists[wid * 64 + lane].i = li;
    }
    __syncthreads();
    if (wid < n - h) {
      const TopEnt o = lists[(wid + h) * 64 + lane];
      wave_list_merge(lv, li, o.v, o.i);
    }
    n = h;
  }
  __syncthreads();
}

}  // namespace mlxf
