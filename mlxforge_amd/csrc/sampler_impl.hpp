#pragma once
// sampler_impl.hpp -- device code of the MI355X (gfx950) batched token
// sampler: the kernels and their launch sequence.  Each sampler_<dtype>.hip
// instantiates it for one logits dtype (the three build in parallel); the host
// side (sampler.hip) calls them through launch_<dtype>.
//
// Replaces the per-row MLX graph of Sampler::sample (src/sample/sampler.cpp:
// 141-166), run once per row by Worker::sample_rows (src/runtime/worker.cpp:
// 448-486), with a short sequence of kernels over all rows of a [B, V] logits
// matrix.  Row r is cut into S slices of L = 256 * EPT logits.  A call is
//
//   k_scan1   one workgroup per slice: the one HBM read of every logit.  Max
//             and lowest-index argmax of z, sum exp(z - max) when a logprob is
//             wanted, the slice minimum and division range for rows that go on
//             to the refine stages, and -- for top_logprobs or top-k <= 63 --
//             the slice's best 64 entries by (z desc, index asc);
//   k_decide1 one workgroup per row: argmax, log-sum-exp, top_logprobs, and
//             for top-k <= 63 the whole selection (k-th value, nucleus, draw)
//             from the merged best-64 lists; every other sampling row gets a
//             plan and goes on the first stage's list;
//   then up to NSTAGE refine stages, each a scan over the slices of the rows on
//   its list and a deciding kernel per row:
//     COUNT   top-k: a 256-bin count histogram of z' over the current bracket;
//     MASS    top-p: a 256-bin histogram of exact fixed-point masses
//             w = exp(z' - max z') (2^-40 units) over the current bracket;
//     GATHER  the bracket's elements themselves (at most CAP per row), resolved
//             exactly by radix selections in LDS;
//     DRAWSUM the kept mass of each slice (temperature-only rows, or top-k sets
//             too large to gather).
//   The first histogram level bins z' on a value grid anchored at the row max
//   (uniform in log-weight, so concentrated rows spread over many bins); later
//   levels take 8-bit digits of the z' key inside the chosen bin.  A row whose
//   cutoff value is known exactly draws: the slice holding u * (kept mass) is
//   found from per-slice kept masses and walked in vocabulary order.  The last
//   stage launched finishes any row still open by running the remaining levels
//   over its slices in its deciding workgroup.
//
// Masses that decide a cutoff are sums of integers, so every result is
// reproducible bit for bit and every level is consistent with the one before.
// Kernels hand data on through the workspace (kernel boundaries order it);
// nothing waits for a workgroup that may not have started.  There is no MFMA
// anywhere: nothing here is a dense contraction.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>

#include "device_common.hpp"
#include "mlxf_sampler.h"

// Per-phase timestamps of the first pass (one record per slice) and the
// deciding kernel (one per row) for a profiling harness that defines
// MLXF_S1_STAMPS (and the arrays they write); no effect otherwise.
#ifdef MLXF_S1_STAMPS
#define MLXF_S1_STAMP(arr, i) \
  if (threadIdx.x == 0) arr[stamp_id * 16 + (i)] = __builtin_amdgcn_s_memrealtime()
#define MLXF_S1_VAL(arr, i, val) \
  if (threadIdx.x == 0) arr[stamp_id * 16 + (i)] = (val)
#define MLXF_S1_STAMP_T(arr, i, t) \
  if (threadIdx.x == (t)) arr[stamp_id * 16 + (i)] = __builtin_amdgcn_s_memrealtime()
#else
#define MLXF_S1_STAMP_T(arr, i, t)
#define MLXF_S1_STAMP(arr, i)
#define MLXF_S1_VAL(arr, i, val)
#endif

namespace mlxf {

enum { KIND_GREEDY = 0, KIND_TEMP = 1, KIND_KLIST = 2, KIND_KHIST = 3, KIND_TOPP = 4 };
enum { PH_DONE = 0, PH_COUNT = 1, PH_MASS = 2, PH_GATHER = 3, PH_DRAWSUM = 4 };
// FL_VGRID: the current level bins z' on the value grid (else key digits kb, sh)
// FL_GALL:  the gather takes every element at or above the bracket's low edge;
//           the top-k selection is finished on the candidates
// FL_TOPP:  a nucleus selection follows the top-k selection
enum { FL_VGRID = 1, FL_GALL = 2, FL_TOPP = 4 };
enum { SL_FAST = 1 };  // slice record flag: the FMA-corrected division is exact for every z

constexpr int LIST = 64;
constexpr int KLIST_MAX = LIST - 1;  // top-k resolved from the best-64 lists
constexpr int NB = 256;              // bins per histogram level
constexpr int CAP = 4096;            // gathered candidates per row (LDS)
constexpr int NSTAGE = 3;            // refine launches per call
constexpr int SERIAL_MAX = 40;       // bound on the levels the last stage runs itself
constexpr int SURV = 64 * 32;        // best-64 survivors of a slice (<= 64 * EPT)
constexpr int SCAP = 128;            // unsorted candidates a slice hands on (else its best 64)
constexpr int SCAP_LOG2 = 7;
constexpr int REC = 8;               // 64-bit words per slice record
constexpr int CBUF = 4096;           // row candidates the deciding workgroup sorts in LDS
constexpr float MASS_LOG2_SPAN = 40.0f;  // weights below 2^-40 quantise to zero


// ------------------------------------------------------------ parameters --

struct Args {
  const void* logits;
  long long row_stride;
  int B, V, K_max, S, L;
  const float* T;
  const int* k;
  const float* p;
  const float* minp;           // [B] or null: min_p
  const int* tlp;
  const float* u;
  int* out_ids;
  float* out_lp;
  int* out_top_ids;
  float* out_top_lp;
  unsigned int* actcnt;        // [4] rows on each stage's list (zero between calls, see below)
  unsigned int* ncand;         // [B] gathered-candidate counters, zero between calls
  unsigned int* actlist;       // [NSTAGE][B] rows still open before each refine stage
  unsigned long long* rec;     // [B*S][REC] slice records
  unsigned long long* list;    // [B*S][SCAP] candidates (z bits, index)
  unsigned long long* rowst;   // [B][8] row plans
  unsigned int* hcnt;          // [B*S][256] histogram counts, cumulative from bin 0 (the top)
  unsigned long long* hmass;   // [B*S][256] histogram masses, cumulative from bin 0
  unsigned long long* above;   // [B*S] kept mass above the bracket (MASS)
  unsigned long long* dsum;    // [B*S] kept mass (DRAWSUM)
  unsigned long long* cand;    // [B][CAP] (z' key, index)
};


// One dtype's launch sequence (defined in sampler_<dtype>.hip).
hipError_t launch_f32(const Args& a, int ept, bool vecok, int nst, hipStream_t st);
hipError_t launch_bf16(const Args& a, int ept, bool vecok, int nst, hipStream_t st);
hipError_t launch_f16(const Args& a, int ept, bool vecok, int nst, hipStream_t st);

// top_logprobs wider than the sampling kernels' lists (TOPK_LIST < K_max;
// defined in filter.hip): every row's top-K (id, logprob), columns past the
// row's K as (-1, -inf), with topk_wide_ws_bytes(B, V, K_max) bytes of
// workspace (256-byte aligned, no initialisation; 0 when K_max <= TOPK_LIST).
constexpr int TOPK_LIST = 64;
size_t topk_wide_ws_bytes(int B, int V, int K_max);
hipError_t launch_topk_wide(const void* logits, int dtype, int B, int V, long long row_stride, const int* tlp,
                            int K_max, int* top_ids, float* top_lp, void* d_ws, hipStream_t st);

namespace {


struct Mode {
  int sampling, kk, topp, K, need_lse, want_lp, kind, need_list, tslow;
  float Tr, pr, u, y, mr;
};

// Per-row parameters with the reference's sentinels and the C ABI's
// sanitisation (src/sample/sampler.h:15-29, src/capi/mlxforge.cpp:43-70).
template <int DT>
__device__ __forceinline__ Mode decode(const Args& a, int r) {
  Mode m;
  const float T = a.T ? a.T[r] : 0.0f;
  m.Tr = round_dt<DT>(T);
  m.sampling = (__builtin_isfinite(T) && T > 0.0f && m.Tr > 0.0f) ? 1 : 0;
  m.y = m.sampling ? 1.0f / m.Tr : 1.0f;  // correctly rounded (IEEE division)
  m.tslow = (m.Tr >= 0x1p-24f && m.Tr <= 0x1p24f) ? 0 : 1;
  const int k = a.k ? a.k[r] : 0;
  m.kk = (m.sampling && k > 0) ? (k < a.V ? k : a.V) : 0;
  const float p = a.p ? a.p[r] : 1.0f;
  m.topp = (m.sampling && p > 0.0f && p < 1.0f) ? 1 : 0;
  m.pr = round_dt<DT>(p);
  // min_p in (0, 1], else off (src/capi/mlxforge.cpp:58), rounded to the
  // logits dtype (src/sample/sampler.cpp:91 multiplies by array(min_p, dtype))
  const float mp = a.minp ? a.minp[r] : 0.0f;
  m.mr = (m.sampling && mp > 0.0f && mp <= 1.0f) ? round_dt<DT>(mp) : 0.0f;
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
  if (!m.sampling)
    m.kind = KIND_GREEDY;
  else if (m.kk > 0)
    m.kind = m.kk <= KLIST_MAX ? KIND_KLIST : KIND_KHIST;
  else
    m.kind = m.topp ? KIND_TOPP : KIND_TEMP;
  m.need_list = (K > 0 || m.kind == KIND_KLIST) ? 1 : 0;
  return m;
}

template <int DT>
__device__ __forceinline__ const void* row_ptr(const Args& a, int r) {
  return static_cast<const char*>(a.logits) +
         static_cast<size_t>(r) * static_cast<size_t>(a.row_stride) * elem_size<DT>();
}

// ------------------------------------------------------ element functions --

// z' = round_dtype(z / Tr) with the quotient correctly rounded (the temperature
// division of src/sample/sampler.cpp:158).  The fast form is Markstein's
// FMA-corrected quotient: with y = RN(1/Tr), q0 = RN(z * y) is within an ulp of
// z / Tr, the remainder z - Tr * q0 is exact by FMA, and RN(q0 + r * y) is the
// correctly rounded quotient (P. Markstein, IBM J. Res. Dev. 34(1), 1990).  It
// is used only when no product, remainder or quotient can leave the normal
// range: 2^-24 <= Tr <= 2^24 and every finite z of the slice has |z| = 0 or
// 2^-96 <= |z| < 2^100 (the slice record's SL_FAST); +-inf passes through.
// Zeros come out as +0, so equal values have equal keys.
template <int DT>
__device__ __forceinline__ float zdiv(float z, float Tr, float y, bool fast) {
  float q;
  if (fast) {
    const float q0 = z * y;
    const float rr = __builtin_fmaf(-q0, Tr, z);
    const float q1 = __builtin_fmaf(rr, y, q0);
    q = rr != rr ? q0 : q1;
  } else {
    q = z / Tr;
  }
  return round_dt<DT>(q) + 0.0f;
}

// Whether |z| lies outside the range the fast division covers (finite z only).
__device__ __forceinline__ bool div_unsafe(float z) {
  const unsigned int az = __float_as_uint(z) & 0x7fffffffu;
  return (az - 1u < 0x0f800000u - 1u) | ((az >= 0x71800000u) & (az < 0x7f800000u));
}

// Monotone key of a z' value: 32 bits for fp32 logits, the 16-bit value's own
// key for bf16 / f16 (z' is a value of the logits dtype).
template <int DT>
constexpr int keybits() {
  return DT == MLXF_DTYPE_F32 ? 32 : 16;
}
template <int DT>
__device__ __forceinline__ unsigned int zkey(float zp) {
  if constexpr (DT == MLXF_DTYPE_F32) {
    return f2key(zp);
  } else if constexpr (DT == MLXF_DTYPE_BF16) {
    return f2key(zp) >> 16;
  } else {
    const unsigned int h = __half_as_ushort(__float2half_rn(zp));
    return (h & 0x8000u) ? (~h & 0xffffu) : (h | 0x8000u);
  }
}
template <int DT>
__device__ __forceinline__ float kval(unsigned int k) {
  if constexpr (DT == MLXF_DTYPE_F32) {
    return key2f(k);
  } else if constexpr (DT == MLXF_DTYPE_BF16) {
    return key2f((k << 16) | ((k & 0x8000u) ? 0u : 0xffffu));
  } else {
    const unsigned int h = (k & 0x8000u) ? (k & 0x7fffu) : (~k & 0xffffu);
    return __half2float(__ushort_as_half(static_cast<unsigned short>(h)));
  }
}
template <int DT>
__device__ __forceinline__ unsigned int key_lo() {  // key of -inf
  return DT == MLXF_DTYPE_F32 ? 0x007fffffu : (DT == MLXF_DTYPE_BF16 ? 0x007fu : 0x03ffu);
}
template <int DT>
__device__ __forceinline__ unsigned int key_hi() {  // key of +inf
  return DT == MLXF_DTYPE_F32 ? 0xff800000u : (DT == MLXF_DTYPE_BF16 ? 0xff80u : 0xfc00u);
}

// log2 of the weight: (z' - Mp) * log2(e) as one FMA with nc = -RN(Mp * log2 e).
// The rounding of nc scales every weight of the row by the same factor (within
// an ulp of 1), which cancels in every mass ratio; min_p, an absolute
// comparison, scales its threshold by the max's own weight (minp_thr).
__device__ __forceinline__ float wlog2(float zp, float nc) { return __builtin_fmaf(zp, LOG2E, nc); }

// w = exp(z' - Mp); for an infinite row max the limit (1 where z' == Mp, else 0).
__device__ __forceinline__ float wfun(float zp, float Mp, float nc, bool minf) {
  return minf ? (zp == Mp ? 1.0f : 0.0f) : __builtin_amdgcn_exp2f(wlog2(zp, nc));
}

// floor(w * 2^40) for w in [0, 1 + 2^-20]: exact fixed-point mass.
__device__ __forceinline__ unsigned long long q40(float w) {
  const float t = w * 256.0f;
  const unsigned int hi = static_cast<unsigned int>(t);
  const float fr = t - floorf(t);
  const unsigned int lo = static_cast<unsigned int>(fr * 4294967296.0f);
  return (static_cast<unsigned long long>(hi) << 32) | lo;
}

// Value-grid bin of a z' (from its log2 weight x <= ~0): 0 at the row max, 255
// at R2 = 255 / span below it and everything further down.  Non-increasing in z'.
__device__ __forceinline__ int vbin_x(float x, float R2) {
  return max(0, min(__float2int_rz(-x * R2), NB - 1));
}

// Smallest k in [lo, hi] with pred(k), for pred false then true over [lo, hi]
// and true at hi: a 64-ary search, one candidate per lane (3 rounds for 16-bit
// keys, 6 for 32-bit).  The whole wave calls it; every lane gets the result.
template <typename PRED>
__device__ __forceinline__ unsigned int wave_search(unsigned int lo, unsigned int hi, PRED pred) {
  const int lane = threadIdx.x & 63;
  while (lo < hi) {
    const unsigned long long span = static_cast<unsigned long long>(hi - lo) + 1ull;
    const unsigned long long step = (span + 63ull) >> 6;
    const unsigned long long k64 = static_cast<unsigned long long>(lo) + step * static_cast<unsigned long long>(lane);
    const unsigned int k = k64 > hi ? hi : static_cast<unsigned int>(k64);
    const unsigned long long bal = __ballot(pred(k));
    if (bal == 0ull) {
      lo = rdl(k, 63) + 1u;
    } else {
      const int f = __ffsll(static_cast<long long>(bal)) - 1;
      const unsigned int kf = rdl(k, f);
      if (f == 0) {
        hi = kf;
        lo = kf;
      } else {
        lo = rdl(k, f - 1) + 1u;
        hi = kf;
      }
    }
  }
  return lo;
}

// wave_search with a guess: one probe of the 64 keys around est (clamped to
// [lo, hi]) settles it when pred turns true inside them and not at the first;
// else the full search.  Whole wave.
template <typename PRED>
__device__ __forceinline__ unsigned int wave_search_near(unsigned int lo, unsigned int hi, unsigned int est, PRED pred) {
  const unsigned int lane = threadIdx.x & 63;
  const unsigned int k0 = est > lo + 32u ? est - 32u : lo;
  const unsigned int k = k0 + lane < hi && k0 + lane >= k0 ? k0 + lane : hi;
  const unsigned long long bal = __ballot(pred(k));
  if (bal != 0ull && (bal & 1ull) == 0ull) return rdl(k, __ffsll(static_cast<long long>(bal)) - 1);
  return wave_search(lo, hi, pred);
}

// Smallest z key whose z' reaches y (z' non-decreasing in z); 0xffffffff if
// none.  Whole wave.
template <int DT>
__device__ __forceinline__ unsigned int gkey(float y, float Tr) {
  if (!(zdiv<DT>(INFINITY, Tr, 1.0f, false) >= y)) return 0xffffffffu;
  auto pred = [&](unsigned int k) { return zdiv<DT>(key2f(k), Tr, 1.0f, false) >= y; };
  // The answer lies within an ulp or two of m * Tr, m the rounding boundary
  // below y (y itself for fp32): one probe of the 64 keys around it settles
  // it when the predicate turns true inside them; else the full search.
  float m = y;
  if constexpr (DT != MLXF_DTYPE_F32) {
    const unsigned int ky = zkey<DT>(y);
    m = ky > key_lo<DT>() ? 0.5f * (y + kval<DT>(ky - 1u)) : y;
  }
  const float est = m * Tr;
  if (__builtin_isfinite(est)) {
    const int lane = threadIdx.x & 63;
    const unsigned int ke = f2key(est);
    const unsigned int k0 = ke > KEY_NEG_INF + 32u ? ke - 32u : KEY_NEG_INF;
    const unsigned int k = min(k0 + static_cast<unsigned int>(lane), KEY_POS_INF);
    const unsigned long long bal = __ballot(pred(k));
    if (bal != 0ull && (bal & 1ull) == 0ull) return rdl(k, __ffsll(static_cast<long long>(bal)) - 1);
  }
  return wave_search(KEY_NEG_INF, KEY_POS_INF, pred);
}

__device__ __forceinline__ unsigned long long pack_ent(float v, int i) {
  return pack2(__float_as_uint(v), static_cast<unsigned int>(i));
}

// (value desc, index asc) as one unsigned order on an entry: the larger key is
// the better entry.  -0 and +0 are equal values, so both take the key of +0
// (and read back as +0).
__device__ __forceinline__ unsigned long long order_key(unsigned long long ent) {
  const float v = __uint_as_float(static_cast<unsigned int>(ent));
  return pack2(0xffffffffu - static_cast<unsigned int>(ent >> 32), f2key(v == 0.0f ? 0.0f : v));
}
__device__ __forceinline__ float order_key_v(unsigned long long k) { return key2f(static_cast<unsigned int>(k >> 32)); }
__device__ __forceinline__ int order_key_i(unsigned long long k) {
  return static_cast<int>(0xffffffffu - static_cast<unsigned int>(k));
}

// min_p (src/sample/sampler.cpp:87-93, after top-p): an element is kept when
// its probability reaches mr times the largest one, i.e. when its weight
// reaches mr times the weight of the row max.  The weight of the max is
// exp2(fma(Mp, log2 e, -RN(Mp * log2 e))), within an ulp of 1 but not 1, so
// the threshold is scaled by it: min_p = 1 then keeps exactly the elements
// whose weight equals the max's, the max among them.
__device__ __forceinline__ float minp_thr(float mr, float Mp, float nc, bool minf) {
  return mr * wfun(Mp, Mp, nc, minf);
}

// Weights are non-decreasing in z', so the kept set is every z' key from the
// smallest one whose weight reaches the threshold.  Whole wave.
template <int DT>
__device__ __forceinline__ unsigned int minp_key(float mr, float Mp, float nc, bool minf) {
  const float thr = minp_thr(mr, Mp, nc, minf);
  return wave_search(key_lo<DT>(), key_hi<DT>(),
                     [&](unsigned int k) { return wfun(kval<DT>(k), Mp, nc, minf) >= thr; });
}

// Sampled id (and its logprob) of row r.
template <int DT>
__device__ __forceinline__ void write_out(const Args& a, int r, int id, double lse, bool want_lp) {
  a.out_ids[r] = id;
  if (a.out_lp) {
    const void* row = row_ptr<DT>(a, r);
    a.out_lp[r] = want_lp ? static_cast<float>(static_cast<double>(ld1<DT>(row, id)) - lse) : NAN;
  }
}


// ----------------------------------------------------------- row plans --

// Row plan words (written by a row's finishing workgroup, read by every
// workgroup of the row in the next stage).
enum {
  RS_PHASE = 0,  // phase | flags << 32
  RS_ZB = 1,     // z-key bracket zlo | zhi << 32 (inclusive)
  RS_DIG = 2,    // key digits: kb | sh << 32
  RS_AUX = 3,    // cabove (participants above the bracket) | fkey (z' key filter) << 32
  RS_GRID = 4,   // Mp bits | R2 bits << 32
  RS_TGT = 5,    // remaining count / mass target inside the bracket (MASS: 0 = not set)
  RS_LSE = 6,    // log-sum-exp of the row (fp64 bits)
  RS_WORDS = 8
};

struct Plan {
  unsigned int phase, flags, zlo, zhi, kb, sh, cabove, fkey;
  float Mp, R2;
  unsigned long long target;
  double lse;
};

__device__ __forceinline__ void plan_store(const Args& a, int r, const Plan& p) {
  unsigned long long* w = a.rowst + static_cast<size_t>(r) * RS_WORDS;
  w[RS_PHASE] = pack2(p.phase, p.flags);
  w[RS_ZB] = pack2(p.zlo, p.zhi);
  w[RS_DIG] = pack2(p.kb, p.sh);
  w[RS_AUX] = pack2(p.cabove, p.fkey);
  w[RS_GRID] = pack2(__float_as_uint(p.Mp), __float_as_uint(p.R2));
  w[RS_TGT] = p.target;
  w[RS_LSE] = static_cast<unsigned long long>(__double_as_longlong(p.lse));
}
__device__ __forceinline__ Plan plan_unpack(const unsigned long long* w) {  // (LDS or global)
  Plan p;
  p.phase = static_cast<unsigned int>(w[RS_PHASE]);
  p.flags = static_cast<unsigned int>(w[RS_PHASE] >> 32);
  p.zlo = static_cast<unsigned int>(w[RS_ZB]);
  p.zhi = static_cast<unsigned int>(w[RS_ZB] >> 32);
  p.kb = static_cast<unsigned int>(w[RS_DIG]);
  p.sh = static_cast<unsigned int>(w[RS_DIG] >> 32);
  p.cabove = static_cast<unsigned int>(w[RS_AUX]);
  p.fkey = static_cast<unsigned int>(w[RS_AUX] >> 32);
  p.Mp = __uint_as_float(static_cast<unsigned int>(w[RS_GRID]));
  p.R2 = __uint_as_float(static_cast<unsigned int>(w[RS_GRID] >> 32));
  p.target = w[RS_TGT];
  p.lse = __longlong_as_double(static_cast<long long>(w[RS_LSE]));
  return p;
}

// First level of a selection over the z' keys >= fkey: the value grid when the
// row max and the span below it are finite and positive, else the top 8 bits of
// the key.  span2 is the span in log2-weight units.
template <int DT>
__device__ __forceinline__ void plan_level1(Plan& p, float span2) {
  if (__builtin_isfinite(p.Mp) && span2 > 0.0f && __builtin_isfinite(span2)) {
    p.flags |= FL_VGRID;
    p.R2 = 255.0f / span2;
  } else {
    p.flags &= ~static_cast<unsigned int>(FL_VGRID);
    p.R2 = 0.0f;
  }
  p.kb = 0u;
  p.sh = static_cast<unsigned int>(keybits<DT>() - 8);
}

// ================================================================ k_scan1 ==
//
// Stage 0, one workgroup per slice: the one HBM read of every logit.

struct alignas(16) S1Lds {
  union alignas(16) {
    TopEnt surv[SURV];         // survivors of a heavy slice
    float stg[THREADS * 32];   // the slice's values, in index order (candidate writes)
  };
  TopEnt lists[WAVES * LIST];  // bitonic fallback for many survivors
  unsigned int klst[WAVES * 64];  // each wave's thread-maximum keys, descending
  float rf[WAVES];
  float rmin[WAVES];
  int ri[WAVES];
  float ramin[WAVES];
  double rd[WAVES];
  double rw[WAVES];
  int rsc[WAVES + 1];
  int ncnt;  // survivors counted so far
  float thv;
  int thi;
};

// Slice s of row r (whole workgroup of THREADS threads), from its loaded bits.
//
// For rows that need their best 64 entries (top_logprobs, top-k <= 63) the
// slice hands on candidates: t_j, the j-th largest thread maximum (j = 64, 32,
// 16, 8, 4, 2, 1), is reached by at least j elements of the slice, so its best
// 64 are all at or above t_64.  Those elements go to the slice's SCAP slots
// unsorted when they fit (the common case: about 73 of 8192 on random rows);
// otherwise (heavy ties) the slice's best 64, sorted.  The t_j go into the
// slice record, where the deciding kernel combines them into a row bound.
// A slice's logits as loaded (raw bits, 8 per 16- or 32-byte load).
template <int DT, int EPT>
struct SliceRaw {
  Raw8<DT> c[EPT / VEC];
};

// (A slice wholly inside the row takes plain vector loads, one per register
// group: no per-lane fallback path whose loads the compiler would wait for
// before reusing the registers.)
template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ void scan1_load(const Args& a, int r, int s, SliceRaw<DT, EPT>& raw) {
  const void* row = row_ptr<DT>(a, r);
  const int beg = s * a.L;
  const int end = min(a.V, beg + a.L);
  const int t8 = static_cast<int>(threadIdx.x) * VEC;
  if (VECOK && end - beg == a.L) {
    const uint4* p = reinterpret_cast<const uint4*>(static_cast<const char*>(row) +
                                                    static_cast<size_t>(beg + t8) * elem_size<DT>());
    constexpr int QPC = CHUNK * Raw8<DT>::NQ / VEC;  // uint4 per CHUNK elements
#pragma unroll
    for (int it = 0; it < EPT / VEC; ++it)
#pragma unroll
      for (int q = 0; q < Raw8<DT>::NQ; ++q) raw.c[it].q[q] = p[it * QPC + q];
  } else {
#pragma unroll
    for (int it = 0; it < EPT / VEC; ++it) load_raw<DT, VECOK>(row, beg + it * CHUNK + t8, end, raw.c[it]);
  }
}

template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ void scan1_body(const Args& a, int r, int s, const SliceRaw<DT, EPT>& raw, S1Lds& sh) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int S = a.S;
  [[maybe_unused]] const int stamp_id = r * S + s;
  // the row's gathered-candidate counter starts at zero (it is first used by a
  // later kernel), so the workspace needs no initialisation and no call
  // depends on what the previous one left
  if (tid == 0 && s == 0) a.ncand[r] = 0u;
  const Mode md = decode<DT>(a, r);
  MLXF_S1_STAMP(mlxf_s1_stamps, 0);
  const int beg = s * a.L;
  const int end = min(a.V, beg + a.L);
  constexpr int NIT = EPT / VEC;
  // rows that reach the refine stages: the division range of the slice, and
  // (top-k rows) its minimum
  const bool refine = md.kind == KIND_TEMP || md.kind == KIND_TOPP || md.kind == KIND_KHIST;

  float v[EPT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) decode8_nan<DT>(raw.c[it], &v[it * VEC]);
  clear_nans(v);
#define MLXF_IDX(e) (beg + ((e) / VEC) * CHUNK + tid * VEC + ((e) % VEC))
  if (md.need_list) {
    // a copy of the values in LDS, where a thread finds its candidates by
    // position (registers cannot be indexed by a lane-varying position)
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      float4* d = reinterpret_cast<float4*>(&sh.stg[it * CHUNK + tid * VEC]);
      d[0] = make_float4(v[it * VEC + 0], v[it * VEC + 1], v[it * VEC + 2], v[it * VEC + 3]);
      d[1] = make_float4(v[it * VEC + 4], v[it * VEC + 5], v[it * VEC + 6], v[it * VEC + 7]);
    }
  }

  static_assert(EPT % 2 == 0, "pairs of elements");
  float tmax = v[0];
#pragma unroll
  for (int e = 1; e < EPT - 1; e += 2) tmax = vmax3(tmax, v[e], v[e + 1]);
  tmax = vmax3(tmax, v[EPT - 1], v[EPT - 1]);
  {
    const float wm = wave_max(tmax);
    if (lane == 0) sh.rf[wid] = wm;
  }
  MLXF_S1_STAMP(mlxf_s1_stamps, 1);
  if (refine) {
    // smallest |z| (the -inf read past the row end is never the smallest) and
    // the slice minimum (with the maximum: the largest finite |z| when neither
    // is infinite)
    float amin = INFINITY;
#pragma unroll
    for (int e = 0; e < EPT; e += 2) amin = vmin3_abs(amin, v[e], v[e + 1]);
    float tmin = INFINITY;
    if (end - beg == a.L) {
#pragma unroll
      for (int e = 0; e < EPT; e += 2) tmin = vmin3(tmin, v[e], v[e + 1]);
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) tmin = fminf(tmin, MLXF_IDX(e) < end ? v[e] : INFINITY);
    }
    amin = wave_min(amin);
    tmin = wave_min(tmin);
    if (lane == 0) {
      sh.ramin[wid] = amin;
      sh.rmin[wid] = tmin;
    }
  }
  if (md.need_list) {
    // each wave's thread-maximum keys, sorted (a thread with no element in the
    // slice counts as key 0, below every key; its first element, at
    // beg + tid * VEC, is its lowest index)
    unsigned int kt = beg + tid * VEC < end ? f2key(tmax) : 0u;
    wave_sort_keys(kt);
    sh.klst[wid * 64 + lane] = kt;
    if (tid == 0) sh.ncnt = 0;
  }
  __syncthreads();
  MLXF_S1_STAMP(mlxf_s1_stamps, 2);
  float zmax = sh.rf[0];
#pragma unroll
  for (int w2 = 1; w2 < WAVES; ++w2) zmax = fmaxf(zmax, sh.rf[w2]);
  {
    // lowest index of the slice max: only threads holding it look
    int tbi = INT_MAX;
    if (tmax == zmax) {
#pragma unroll
      for (int e = EPT - 1; e >= 0; --e)
        if (v[e] == zmax && MLXF_IDX(e) < end) tbi = MLXF_IDX(e);
    }
    const int wa = wave_min(tbi);
    if (lane == 0) sh.ri[wid] = wa;
  }
  if (md.need_lse) {
    float t = 0.0f;
    if (__builtin_isfinite(zmax)) {
      // entries past the row end read as -inf and weigh 0
#pragma unroll
      for (int e = 0; e < EPT; ++e) t += __builtin_amdgcn_exp2f((v[e] - zmax) * LOG2E);
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e)
        if (MLXF_IDX(e) < end) t += wexp(v[e], zmax);
    }
    const double ws = wave_sum(static_cast<double>(t));
    if (lane == 0) sh.rd[wid] = ws;
  }
  if (md.kind == KIND_TOPP && md.need_list) {
    // top-p rows with a list: the slice's weights relative to its own
    // largest z' (the weight function of the draw with the slice's offset
    // ncs in place of the row's), from which the deciding kernel bounds the
    // row's total mass.  (Entries past the row end read as -inf and weigh 0.)
    const float mps = zdiv<DT>(zmax, md.Tr, md.y, true);
    float t = 0.0f;
    if (__builtin_isfinite(mps)) {
      const float ncs = -(mps * LOG2E);
#pragma unroll
      for (int e = 0; e < EPT; ++e) t += __builtin_amdgcn_exp2f(wlog2(zdiv<DT>(v[e], md.Tr, md.y, true), ncs));
    }
    const double ws = wave_sum(static_cast<double>(t));
    if (lane == 0) sh.rw[wid] = ws;
  }
  MLXF_S1_STAMP(mlxf_s1_stamps, 6);
  unsigned int msk = 0u;  // the thread's survivors (elements at or above t_64)
  int pos0 = 0;           // ... their first slot
  unsigned int t64 = 0u, t32 = 0u, t16 = 0u, t8 = 0u, t4 = 0u, t2 = 0u, t1 = 0u;
  if (md.need_list) {
    // the slice's 64 largest thread maxima, descending, in every wave (two
    // independent merges, then one)
    static_assert(WAVES == 4, "four wave lists");
    unsigned int mk = sh.klst[lane], mk2 = sh.klst[128 + lane];
    wave_merge_keys(mk, sh.klst[64 + lane]);
    wave_merge_keys(mk2, sh.klst[192 + lane]);
    wave_merge_keys(mk, mk2);
    t64 = rdl(mk, 63);
    t32 = rdl(mk, 31);
    t16 = rdl(mk, 15);
    t8 = rdl(mk, 7);
    t4 = rdl(mk, 3);
    t2 = rdl(mk, 1);
    t1 = rdl(mk, 0);
    MLXF_S1_STAMP(mlxf_s1_stamps, 7);
    // survivors: every element at or above t_64.  The float compare keeps -0
    // with +0, which (value desc, index asc) order ties.
    const float thf = t64 <= KEY_NEG_INF ? -INFINITY : key2f(t64);
    // entries past the row end read as -inf: they need the bounds check only
    // when theta is -inf
    const bool nochk = end - beg == a.L || thf > -INFINITY;
    static_assert(EPT <= 32, "one mask bit per element");
    if (nochk) {
#pragma unroll
      for (int e = 0; e < EPT; ++e) msk |= (v[e] >= thf ? 1u : 0u) << e;
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) msk |= (((MLXF_IDX(e) < end) & (v[e] >= thf)) ? 1u : 0u) << e;
    }
    const int mine = __builtin_popcount(msk);
    MLXF_S1_STAMP(mlxf_s1_stamps, 8);
    // slots: a DPP scan within the wave and one LDS atomic per wave for its
    // base, no barrier.  (The waves' order varies from run to run, and with it
    // the order of the slots; every reader orders candidates by value and
    // index.)
    const int incl = wave_incl_scan_dpp(mine);
    int wbase = 0;
    if (lane == 63) wbase = __hip_atomic_fetch_add(&sh.ncnt, incl, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    pos0 = __builtin_amdgcn_readlane(wbase, 63) + incl - mine;
    MLXF_S1_STAMP(mlxf_s1_stamps, 9);
    // unsorted, straight into the slice's slots, one pass per candidate of
    // the thread (usually none or one); a slice found to hold more than SCAP
    // rewrites its slots below
    unsigned long long* dst = a.list + (static_cast<size_t>(r) * S + s) * SCAP;
    unsigned int m = msk;
    int pos = pos0;
    while (m) {
      const int e = __builtin_ctz(m);
      m &= m - 1u;
      const int off = (e / VEC) * CHUNK + tid * VEC + (e % VEC);
      if (pos < SCAP) dst[pos] = pack_ent(sh.stg[off], beg + off);
      ++pos;
    }
  }
  MLXF_S1_STAMP(mlxf_s1_stamps, 3);
  __syncthreads();
  MLXF_S1_STAMP(mlxf_s1_stamps, 4);
  int zarg = sh.ri[0];
#pragma unroll
  for (int w2 = 1; w2 < WAVES; ++w2) zarg = min(zarg, sh.ri[w2]);
  double lse_s = 0.0;
  if (md.need_lse) {
    lse_s = sh.rd[0];
#pragma unroll
    for (int w2 = 1; w2 < WAVES; ++w2) lse_s += sh.rd[w2];
  }
  float zmin = 0.0f;
  unsigned int sfl = 0u;
  if (refine) {
    float amin = sh.ramin[0];
    zmin = sh.rmin[0];
#pragma unroll
    for (int w2 = 1; w2 < WAVES; ++w2) {
      amin = fminf(amin, sh.ramin[w2]);
      zmin = fminf(zmin, sh.rmin[w2]);
    }
    // the FMA-corrected division is exact when every nonzero |z| >= 2^-96 and
    // every finite |z| < 2^100: here, when every |z| >= 2^-96 and the slice's
    // maximum and minimum are both below 2^100 in magnitude (a slice holding a
    // zero or an infinity divides exactly)
    sfl = (amin >= 0x1p-96f && fabsf(zmax) < 0x1p100f && fabsf(zmin) < 0x1p100f)
              ? static_cast<unsigned int>(SL_FAST)
              : 0u;
  }
  // more than SCAP survivors (heavy ties at t_64): the slice hands on its
  // best 64, sorted, in place of the slots written above
  int nsurv = md.need_list ? sh.ncnt : 0;
  const bool heavy = nsurv > SCAP;
  if (heavy) {
    if (nsurv <= SURV) {
      // the survivors into LDS, at the slots counted above
      int pos = pos0;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        if ((msk >> e) & 1u) {
          sh.surv[pos].v = v[e];
          sh.surv[pos].i = MLXF_IDX(e);
          ++pos;
        }
      }
    } else {
      // the exact 64th best thread maximum instead, which at most 64 * EPT
      // elements reach: bitonic sort of each wave's 64 and a tree merge; with
      // fewer than 64 threads holding elements it is the sentinel and every
      // element survives
      float lv = -INFINITY;
      int li = INT_MAX;
#pragma unroll
      for (int e = EPT - 1; e >= 0; --e)
        if (v[e] == tmax && MLXF_IDX(e) < end) li = MLXF_IDX(e);
      if (li != INT_MAX) lv = tmax;
      wave_sort(lv, li);
      tree_merge(lv, li, sh.lists, WAVES);
      if (tid == LIST - 1) {
        sh.thv = lv;
        sh.thi = li;
      }
      __syncthreads();
      const float tv = sh.thv;
      const int ti = sh.thi;
      int mine2 = 0;
#pragma unroll
      for (int e = 0; e < EPT; ++e) mine2 += (MLXF_IDX(e) < end && !better(tv, ti, v[e], MLXF_IDX(e))) ? 1 : 0;
      int pos = block_excl_scan_dpp<int>(mine2, sh.rsc, &nsurv);
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const int i = MLXF_IDX(e);
        if (i < end && !better(tv, ti, v[e], i)) {
          sh.surv[pos].v = v[e];
          sh.surv[pos].i = i;
          ++pos;
        }
      }
    }
    __syncthreads();
    // 64-entry chunks sorted by the waves and merged
    unsigned long long* dst = a.list + (static_cast<size_t>(r) * S + s) * SCAP;
    const int nch = (nsurv + LIST - 1) / LIST;
    float sv = -INFINITY;
    int si = INT_MAX;
    for (int ch = wid; ch < nch; ch += WAVES) {
      const int c = ch * LIST + lane;
      float cv = -INFINITY;
      int ci = INT_MAX;
      if (c < nsurv) {
        cv = sh.surv[c].v;
        ci = sh.surv[c].i;
      }
      wave_sort(cv, ci);
      wave_list_merge(sv, si, cv, ci);
    }
    if (nch > 1) tree_merge(sv, si, sh.lists, nch < WAVES ? nch : WAVES);
    if (wid == 0) dst[lane] = pack_ent(sv, si);
  }
#undef MLXF_IDX
  if (tid == 0) {
    unsigned long long* rp = a.rec + (static_cast<size_t>(r) * S + s) * REC;
    rp[0] = pack2(__float_as_uint(zmax), static_cast<unsigned int>(zarg));
    rp[1] = pack2(__float_as_uint(zmin), sfl);
    rp[2] = static_cast<unsigned long long>(__double_as_longlong(lse_s));
    if (md.need_list) {
      rp[3] = pack2(t64, t32);
      rp[4] = pack2(t16, t8);
      rp[5] = pack2(t4, static_cast<unsigned int>(heavy ? LIST : nsurv));
      rp[6] = pack2(t2, t1);
    }
    if (md.kind == KIND_TOPP && md.need_list) {
      // the slice's weight sum; 0 for a slice of -inf only, NaN (no bound)
      // when its max is +inf
      double ws = sh.rw[0];
#pragma unroll
      for (int w2 = 1; w2 < WAVES; ++w2) ws += sh.rw[w2];
      if (!__builtin_isfinite(zmax)) ws = zmax < 0.0f ? 0.0 : static_cast<double>(NAN);
      rp[7] = static_cast<unsigned long long>(__double_as_longlong(ws));
    }
  }
  MLXF_S1_STAMP(mlxf_s1_stamps, 5);
}

// Slice s of row r (whole workgroup of THREADS threads).  Also called slice
// after slice by the fallback kernel of the row-histogram path.
template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ void scan1_slice(const Args& a, int r, int s, S1Lds& sh) {
  SliceRaw<DT, EPT> raw;
  scan1_load<DT, EPT, VECOK>(a, r, s, raw);
  scan1_body<DT, EPT, VECOK>(a, r, s, raw, sh);
}

template <int DT, int EPT, bool VECOK>
__global__ __launch_bounds__(THREADS) void k_scan1(Args a) {
  __shared__ S1Lds sh;
  const int bid = static_cast<int>(blockIdx.x);
  const int r = bid / a.S, s = bid - r * a.S;
  // a new call: the stage lists of the previous call (whatever number of
  // stages it launched) are spent
  if (bid == 0 && threadIdx.x < NSTAGE) a.actcnt[threadIdx.x] = 0u;
  scan1_slice<DT, EPT, VECOK>(a, r, s, sh);
}

// ============================================================== k_decide1 ==
//
// Stage 0, one workgroup per row: argmax, log-sum-exp, top_logprobs, top-k <= 63
// from the merged best-64 lists; a plan for every other sampling row.

struct D1Lds {
  unsigned long long sv[CBUF];  // the row's candidates at or above theta, as order keys
  alignas(16) unsigned int thr[7 * MAX_S];  // [j][s]: t_64, t_32, t_16, t_8, t_4, t_2, t_1 of each slice
  int sn[MAX_S];                // per slice: candidates handed on
  int ncnt;                     // candidates gathered
  unsigned int thw[WAVES];      // each wave's best theta
  TopEnt lists[WAVES * LIST];
  TopEnt mlist[LIST];
  float szmax[MAX_S];
  int szarg[MAX_S];
  float szmin[MAX_S];
  double slse[MAX_S];
  double swsum[MAX_S];  // top-p rows: each slice's weight sum relative to its own max
  float zmax, zmin;
  int zarg;
  double lse;
  double wlo, whi;      // top-p rows: bounds on the row's total fixed-point mass
  int wok;              // ... usable
  int sel[4];
  unsigned long long kl_tu;  // two-wave top-k: the draw target
  int kl_nk;                 // ... entries kept (negated when their weights are all 0)
};

// Top-k <= 63 from the row's merged best-64 list, by one wave.  Returns false
// when the list may miss elements tied at the k-th value of z' (the caller then
// plans a full top-k selection).  The nucleus and the draw follow
// src/sample/sampler.cpp:63-85,165 on the list: (z' desc, index asc) order,
// keep while the mass before an entry is < p * W_k, inverse CDF in vocabulary
// order.
template <int DT>
__device__ __forceinline__ bool klist_resolve(const Mode& md, float Mp, const TopEnt* ml, int* id_out) {
  const int lane = threadIdx.x & 63;
  const float lv = ml[lane].v;
  const int li = ml[lane].i;
  const bool real = li != INT_MAX;
  const float zp = real ? zdiv<DT>(lv, md.Tr, md.y, false) : -INFINITY;
  const float tau = rdl(zp, md.kk - 1);
  const int last_i = rdl(li, LIST - 1);
  const float last_zp = rdl(zp, LIST - 1);
  if (last_i != INT_MAX && !(last_zp < tau)) return false;
  const bool in_k = real && zp >= tau;
  float sv = in_k ? zp : -INFINITY;
  int si = in_k ? li : INT_MAX;
  // (z' desc, index asc): the list is in (z desc, index asc) order and z' is
  // non-decreasing in z, so only entries whose z' the rounding made equal can be
  // out of order -- and then some neighbouring pair is
  const float nsv = __shfl_down(sv, 1, 64);
  const int nsi = __shfl_down(si, 1, 64);
  if (__ballot(lane < 63 && sv == nsv && si > nsi)) wave_sort(sv, si);
  const bool k1 = si != INT_MAX;
  const float nc = -(Mp * LOG2E);
  const bool minf = !__builtin_isfinite(Mp);
  // masses in 2^-40 units: each below 2^41, so every sum of 64 is an exact double
  const float wv = k1 ? wfun(sv, Mp, nc, minf) : 0.0f;
  const double w = static_cast<double>(q40(wv));
  const double incl = wave_incl_scan_dpp(w);
  const double Wk = rdl(incl, 63);
  bool keep = k1;
  if (md.topp) {
    const double PW = ceil(static_cast<double>(md.pr) * Wk);
    keep = k1 && (incl - w) < PW;
  }
  if (md.mr > 0.0f) keep = keep && wv >= minp_thr(md.mr, Mp, nc, minf);  // min_p, after top-p
  const double wf = keep ? w : 0.0;
  const double Wf = wave_sum(wf);
  unsigned long long Tu = static_cast<unsigned long long>(static_cast<double>(md.u) * Wf);
  if (Wf == 0.0)
    Tu = 0;
  else if (static_cast<double>(Tu) >= Wf)
    Tu = static_cast<unsigned long long>(Wf) - 1;
  // the kept entries in vocabulary order and their running mass
  int ki = keep ? si : INT_MAX;
  double kw = wf;
  wave_sort_idx(ki, kw);
  const double cum = wave_incl_scan_dpp(kw);
  const int cand = wave_min((ki != INT_MAX && (Wf == 0.0 || (kw > 0.0 && cum > static_cast<double>(Tu)))) ? ki : INT_MAX);
  *id_out = cand == INT_MAX ? rdl(si, 0) : cand;
  return true;
}

// The part of klist_resolve both waves of the two-wave form compute: the list's
// top-k entries in (z' desc, index asc) order (sv, si; (-inf, INT_MAX) past
// them) and their fixed-point masses.  False as for klist_resolve.
template <int DT>
__device__ __forceinline__ bool klist_prep(const Mode& md, float Mp, const TopEnt* ml, float& sv, int& si,
                                           float& wv, double& w) {
  const int lane = threadIdx.x & 63;
  const float lv = ml[lane].v;
  const int li = ml[lane].i;
  const bool real = li != INT_MAX;
  const float zp = real ? zdiv<DT>(lv, md.Tr, md.y, false) : -INFINITY;
  const float tau = rdl(zp, md.kk - 1);
  const int last_i = rdl(li, LIST - 1);
  const float last_zp = rdl(zp, LIST - 1);
  if (last_i != INT_MAX && !(last_zp < tau)) return false;
  const bool in_k = real && zp >= tau;
  sv = in_k ? zp : -INFINITY;
  si = in_k ? li : INT_MAX;
  const float nsv = __shfl_down(sv, 1, 64);
  const int nsi = __shfl_down(si, 1, 64);
  if (__ballot(lane < 63 && sv == nsv && si > nsi)) wave_sort(sv, si);
  const float nc = -(Mp * LOG2E);
  wv = si != INT_MAX ? wfun(sv, Mp, nc, !__builtin_isfinite(Mp)) : 0.0f;
  w = static_cast<double>(q40(wv));
  return true;
}

// For a top-p row: every real entry of the row's best-64 list in (z' desc,
// index asc) order (sv, si; (-inf, INT_MAX) past them), their weights and
// fixed-point masses, and the z' and index of the list's last entry (every
// element outside the list has z' at most that z').
template <int DT>
__device__ __forceinline__ void plist_prep(const Mode& md, float Mp, const TopEnt* ml, float& sv, int& si, float& wv,
                                           double& w, float& last_zp, int& last_i) {
  const int lane = threadIdx.x & 63;
  const float lv = ml[lane].v;
  const int li = ml[lane].i;
  const bool real = li != INT_MAX;
  const float zp = real ? zdiv<DT>(lv, md.Tr, md.y, false) : -INFINITY;
  last_i = rdl(li, LIST - 1);
  last_zp = rdl(zp, LIST - 1);
  sv = zp;
  si = real ? li : INT_MAX;
  const float nsv = __shfl_down(sv, 1, 64);
  const int nsi = __shfl_down(si, 1, 64);
  if (__ballot(lane < 63 && sv == nsv && si > nsi)) wave_sort(sv, si);
  const float nc = -(Mp * LOG2E);
  wv = si != INT_MAX ? wfun(sv, Mp, nc, !__builtin_isfinite(Mp)) : 0.0f;
  w = static_cast<double>(q40(wv));
}

// Put row r (its next phase in the high half) on the list of refine stage
// `stage` (0-based).
__device__ __forceinline__ void enlist(const Args& a, int stage, int r, unsigned int phase) {
  const unsigned int pos =
      __hip_atomic_fetch_add(a.actcnt + stage, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  a.actlist[static_cast<size_t>(stage) * a.B + pos] = static_cast<unsigned int>(r) | (phase << 16);
}

// =================================================================== stages ==

// Shared memory of a stage's slice pass (kept small: it bounds the occupancy
// of the streaming kernels).
struct SLds {
  unsigned long long pw[RS_WORDS];   // the row plan as read
  unsigned int hc[NB + 64];          // slice histogram: counts (+ one unread slot per lane)
  unsigned long long hm[NB + 64];    // slice histogram: masses (+ one unread slot per lane)
  unsigned long long ru[WAVES + 1];
  unsigned int rv[WAVES + 1];
  unsigned int ncand;
};
// ... and of a deciding workgroup.
struct RLds {
  SLds sl;
  unsigned long long cand[CAP];      // gathered candidates (z' key | index << 32)
  unsigned long long cmq[CAP];       // ... and their fixed-point masses
  unsigned long long kept[MAX_S];    // per-slice kept mass
  unsigned int tcnt[MAX_S];          // per-slice ties / counts
  int ri[WAVES + 1];
  int sel[8];
  unsigned long long selu[8];
  unsigned int kmin, kmax, ncand;
  int found;
  float wz[64];                      // the draw's run of elements (walk)
  unsigned long long wex;
  unsigned int wrk;
  int wbase;
};

// ---- a slice's histogram in the common case (the FMA-corrected division, a
// finite row max) as straight-line code, so the elements' exps, conversions and
// LDS atomics overlap: the flags that are uniform over the slice -- MASS, the
// value grid VG, and FULL (no bracket or row-end test needed) -- are template
// parameters, and an element that adds nothing (outside the bracket or the row,
// or of zero mass in the MASS phase) goes to its lane's own slot past the NB
// bins, which nothing reads.  Bins and masses are those of the generic path.
template <int DT, int EPT, bool MASS, bool VG, bool FULL>
__device__ __forceinline__ void hist_fast(const float (&v)[EPT], const Mode& md, const Plan& pl, float nc, int beg,
                                          int end, SLds& sh) {
  const int tid = threadIdx.x, lane = tid & 63;
#pragma unroll
  for (int e = 0; e < EPT; ++e) {
    const float zp = zdiv<DT>(v[e], md.Tr, md.y, true);
    const float x = wlog2(zp, nc);
    bool ok = true;
    if constexpr (!FULL) {
      const unsigned int zk = f2key(v[e]);
      const int i = beg + (e / VEC) * CHUNK + tid * VEC + (e % VEC);
      ok = i < end && zk >= pl.zlo && zk <= pl.zhi;
    }
    unsigned long long q = 0;
    if constexpr (MASS) {
      q = q40(__builtin_amdgcn_exp2f(x));
      ok = ok && q != 0ull;
    }
    int bin;
    if constexpr (VG)
      bin = vbin_x(x, pl.R2);
    else
      bin = max(0, NB - 1 - static_cast<int>(min((zkey<DT>(zp) - pl.kb) >> pl.sh, 255u)));
    bin = ok ? bin : NB + lane;
    atomicAdd(&sh.hc[bin], 1u);
    if constexpr (MASS) atomicAdd(&sh.hm[bin], q);
  }
}

template <int DT, int EPT, bool MASS>
__device__ __forceinline__ void hist_fast_any(bool vg, bool full, const float (&v)[EPT], const Mode& md,
                                              const Plan& pl, float nc, int beg, int end, SLds& sh) {
  if (vg) {
    if (full)
      hist_fast<DT, EPT, MASS, true, true>(v, md, pl, nc, beg, end, sh);
    else
      hist_fast<DT, EPT, MASS, true, false>(v, md, pl, nc, beg, end, sh);
  } else {
    if (full)
      hist_fast<DT, EPT, MASS, false, true>(v, md, pl, nc, beg, end, sh);
    else
      hist_fast<DT, EPT, MASS, false, false>(v, md, pl, nc, beg, end, sh);
  }
}

// ---- one slice of one stage: the histogram, the gathered elements or the kept
// mass of slice s of row r under the plan in sh.pw.  Results go to the
// workspace with plain stores (read by the next kernel, or -- in the last
// stage -- by this workgroup after a full wait and a barrier).
template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ void slice_stage(const Args& a, int r, int s, const Plan& pl, SLds& sh) {
  const int tid = threadIdx.x;
  const Mode md = decode<DT>(a, r);
  const void* row = row_ptr<DT>(a, r);
  const int beg = s * a.L;
  const int end = min(a.V, beg + a.L);
  constexpr int NIT = EPT / VEC;
  const unsigned int sfl = static_cast<unsigned int>(a.rec[(static_cast<size_t>(r) * a.S + s) * REC + 1] >> 32);
  const bool fast = !md.tslow && (sfl & SL_FAST);
  const float Mp = pl.Mp;
  const float nc = -(Mp * LOG2E);
  const bool minf = !__builtin_isfinite(Mp);
  const bool vgrid = (pl.flags & FL_VGRID) != 0;
  const unsigned int zlo = pl.zlo, zhi = pl.zhi;

  float v[EPT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) load8_nan<DT, VECOK>(row, beg + it * CHUNK + tid * VEC, end, &v[it * VEC]);
  clear_nans(v);  // NaN reads as -inf
#define MLXF_IDX(e) (beg + ((e) / VEC) * CHUNK + tid * VEC + ((e) % VEC))

  if (pl.phase == PH_COUNT || pl.phase == PH_MASS) {
    const bool mass = pl.phase == PH_MASS;
    for (int b = tid; b < NB; b += THREADS) {
      sh.hc[b] = 0u;
      sh.hm[b] = 0ull;
    }
    __syncthreads();
    auto add = [&](float z) {
      const float zp = zdiv<DT>(z, md.Tr, md.y, fast);
      const float x = wlog2(zp, nc);
      unsigned long long q = 0;
      if (mass) q = q40(minf ? (zp == Mp ? 1.0f : 0.0f) : __builtin_amdgcn_exp2f(x));
      if (!mass || q) {
        const int bin = vgrid ? vbin_x(x, pl.R2)
                              : max(0, NB - 1 - static_cast<int>(min((zkey<DT>(zp) - pl.kb) >> pl.sh, 255u)));
        atomicAdd(&sh.hc[bin], 1u);
        if (mass) atomicAdd(&sh.hm[bin], q);
      }
    };
    // the first level brackets every key; entries past the row end read as
    // -inf, which weigh nothing (MASS) -- so no per-element test is needed
    const bool full = zlo <= KEY_NEG_INF && zhi >= KEY_POS_INF && (mass || end - beg == a.L);
    if (fast && !minf) {
      if (mass)
        hist_fast_any<DT, EPT, true>(vgrid, full, v, md, pl, nc, beg, end, sh);
      else
        hist_fast_any<DT, EPT, false>(vgrid, full, v, md, pl, nc, beg, end, sh);
    } else if (full) {
#pragma unroll
      for (int e = 0; e < EPT; ++e) add(v[e]);
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const unsigned int zk = f2key(v[e]);
        if (MLXF_IDX(e) < end && zk >= zlo && zk <= zhi) add(v[e]);
      }
    }
    __syncthreads();
    // cumulative from the top bin down: the deciding step reads a bin's total
    // and everything above it in one word
    const size_t o = (static_cast<size_t>(r) * a.S + s) * NB;
    const int ci = static_cast<int>(sh.hc[tid]);
    int ctot;
    a.hcnt[o + tid] = static_cast<unsigned int>(block_excl_scan_dpp<int>(ci, reinterpret_cast<int*>(sh.rv), &ctot) + ci);
    if (mass) {
      const unsigned long long mi = sh.hm[tid];
      unsigned long long mtot;
      a.hmass[o + tid] = block_excl_scan_dpp<unsigned long long>(mi, sh.ru, &mtot) + mi;
    }
  } else if (pl.phase == PH_GATHER) {
    // the slice's elements in the bracket: one reservation per workgroup
    unsigned int mine = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const unsigned int zk = f2key(v[e]);
      mine += (MLXF_IDX(e) < end && zk >= zlo && zk <= zhi) ? 1u : 0u;
    }
    int total;
    int pos = block_excl_scan_dpp<int>(static_cast<int>(mine), reinterpret_cast<int*>(sh.rv), &total);
    if (tid == 0)
      sh.ncand = total ? __hip_atomic_fetch_add(a.ncand + r, static_cast<unsigned int>(total), __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT)
                       : 0u;
    __syncthreads();
    pos += static_cast<int>(sh.ncand);
    unsigned long long* dst = a.cand + static_cast<size_t>(r) * CAP;
    if (mine) {
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const unsigned int zk = f2key(v[e]);
        if (MLXF_IDX(e) < end && zk >= zlo && zk <= zhi) {
          const float zp = zdiv<DT>(v[e], md.Tr, md.y, fast);
          if (pos < CAP) dst[pos] = pack2(zkey<DT>(zp), static_cast<unsigned int>(MLXF_IDX(e)));
          ++pos;
        }
      }
    }
  } else if (pl.phase == PH_DRAWSUM) {
    // kept: z' keys from fkey (the bracket holds them; a min_p threshold can
    // fall inside the bracket's edge values)
    unsigned long long t = 0;
    const bool fk = pl.fkey > key_lo<DT>();
    if (fast && !minf) {
      // straight-line: every element's mass computed, the kept ones summed
      // (with no threshold, key >= 0 keeps all)
      const unsigned int fke = fk ? pl.fkey : 0u;
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const unsigned int zk = f2key(v[e]);
        const float zp = zdiv<DT>(v[e], md.Tr, md.y, true);
        const unsigned long long q = q40(__builtin_amdgcn_exp2f(wlog2(zp, nc)));
        const bool keep = MLXF_IDX(e) < end && zk >= zlo && zk <= zhi && zkey<DT>(zp) >= fke;
        t += keep ? q : 0ull;
      }
    } else {
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const unsigned int zk = f2key(v[e]);
        if (MLXF_IDX(e) < end && zk >= zlo && zk <= zhi) {
          const float zp = zdiv<DT>(v[e], md.Tr, md.y, fast);
          if (!fk || zkey<DT>(zp) >= pl.fkey) t += q40(wfun(zp, Mp, nc, minf));
        }
      }
    }
    t = block_sum<unsigned long long>(t, sh.ru);
    if (tid == 0) a.dsum[static_cast<size_t>(r) * a.S + s] = t;
  }
#undef MLXF_IDX
}

// ---- the draw: walk slice s in vocabulary order; kept elements are those with
// z' key > tau, and the first tie_lim (in index order) of those equal to tau.
// Returns the first kept element at which the running kept mass exceeds rem.
template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ int walk(const Args& a, int r, int s, float Mp, unsigned long long rem, unsigned int tau,
                    unsigned int tie_lim, RLds& sh) {
  const int tid = threadIdx.x;
  const Mode md = decode<DT>(a, r);
  const void* row = row_ptr<DT>(a, r);
  const int b0 = s * a.L, e0 = min(a.V, b0 + a.L);
  const int my0 = b0 + tid * EPT;
  const unsigned int sfl = static_cast<unsigned int>(a.rec[(static_cast<size_t>(r) * a.S + s) * REC + 1] >> 32);
  const bool fast = !md.tslow && (sfl & SL_FAST);
  const float nc = -(Mp * LOG2E);
  const bool minf = !__builtin_isfinite(Mp);
  // z' values are never -0 (zdiv), so the key of -0 keeps every z' >= +0: as a
  // value threshold that is +0 with every tie kept
  float tauf = kval<DT>(tau);
  unsigned int lim = tie_lim;
  if (tau == (1u << (keybits<DT>() - 1)) - 1u) {
    tauf = 0.0f;
    lim = 0xffffffffu;
  }
  // thread t owns EPT consecutive elements, held as z' values
  float zp[EPT];
#pragma unroll
  for (int it = 0; it < EPT / VEC; ++it) load8<DT, VECOK>(row, my0 + it * VEC, e0, &zp[it * VEC]);
  // the division form chosen once for the run, so each loop is straight-line
  if (fast) {
#pragma unroll
    for (int e = 0; e < EPT; ++e) zp[e] = zdiv<DT>(zp[e], md.Tr, md.y, true);
  } else {
#pragma unroll
    for (int e = 0; e < EPT; ++e) zp[e] = zdiv<DT>(zp[e], md.Tr, md.y, false);
  }
  // rank of my first tie at tau among the slice's ties (all ties kept: none)
  const bool all_ties = lim == 0xffffffffu;
  int tex = 0;
  if (!all_ties) {
    int nt = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) nt += ((my0 + e < e0) & (zp[e] == tauf)) ? 1 : 0;
    int ttot;
    tex = block_excl_scan_dpp<int>(nt, sh.ri, &ttot);
  }
  unsigned long long qs = 0;
  int last = -1;
  {
    // straight-line over the elements (bitwise tests, every weight computed
    // and masked): a branch per test would run the elements one by one, each
    // waiting for its exp
    unsigned int rk = static_cast<unsigned int>(tex);
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const bool valid = my0 + e < e0;
      const bool tie = valid & (zp[e] == tauf);
      const bool kept = valid & ((zp[e] > tauf) | (tie & (rk < lim)));
      rk += tie ? 1u : 0u;
      const unsigned long long qv = q40(wfun(zp[e], Mp, nc, minf));
      const unsigned long long q = kept ? qv : 0ull;
      qs += q;
      last = q > 0 ? my0 + e : last;
    }
  }
  if (tid == 0) sh.found = -1;
  unsigned long long tot;
  const unsigned long long ex = block_excl_scan_dpp<unsigned long long>(qs, sh.sl.ru, &tot);
  if (ex <= rem && rem < ex + qs) {
    // the one thread whose run holds the draw hands its elements to wave 0
#pragma unroll
    for (int e = 0; e < EPT; ++e) sh.wz[e] = zp[e];
    sh.wex = ex;
    sh.wrk = static_cast<unsigned int>(tex);
    sh.wbase = my0;
    sh.found = -2;
  }
  __syncthreads();
  if (tid < 64 && sh.found == -2) {
    // one element per lane: running kept mass in index order, first past rem
    const int lane = tid;
    const int idx = sh.wbase + lane;
    const bool valid = lane < EPT && idx < e0;
    const float z = lane < EPT ? sh.wz[lane] : -INFINITY;
    const bool tie = valid && z == tauf;
    const unsigned long long tb = __ballot(tie);
    const unsigned int rk = sh.wrk + __builtin_amdgcn_mbcnt_hi(static_cast<unsigned int>(tb >> 32),
                                                               __builtin_amdgcn_mbcnt_lo(static_cast<unsigned int>(tb), 0u));
    const bool kept = valid && (z > tauf || (tie && rk < lim));
    const unsigned long long q = kept ? q40(wfun(z, Mp, nc, minf)) : 0ull;
    const unsigned long long c = sh.wex + wave_incl_scan_dpp(q);
    const int pk = wave_min((q > 0 && c > rem) ? idx : INT_MAX);
    if (lane == 0) sh.found = pk == INT_MAX ? -1 : pk;
  }
  __syncthreads();
  int id = sh.found;
  if (id < 0) {  // rem reached no element: the last kept element with positive mass
    const int lm = wave_max(last);
    if ((tid & 63) == 0) sh.ri[tid >> 6] = lm;
    __syncthreads();
    if (tid == 0) {
      int m = -1;
      for (int w2 = 0; w2 < WAVES; ++w2) m = max(m, sh.ri[w2]);
      sh.found = m < 0 ? b0 : m;
    }
    __syncthreads();
    id = sh.found;
  }
  __syncthreads();
  return id;
}

// Pick the slice holding the draw from per-slice kept masses sh.kept[0..S) and
// walk it.  sh.tcnt[s] holds the kept ties of slice s unless all ties are kept.
template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ int draw(const Args& a, int r, const Mode& md, float Mp, unsigned int tau, bool all_ties,
                    RLds& sh) {
  const int tid = threadIdx.x;
  const int S = a.S;
  if (tid < 64) {
    // lane t: slice t's kept mass and the running sum up to it (S <= 64)
    const int lane = tid;
    const unsigned long long kt = lane < S ? sh.kept[lane] : 0ull;
    const unsigned long long inc = wave_incl_scan_dpp(kt);
    const unsigned long long W = rdl(inc, 63);
    unsigned long long Tu = static_cast<unsigned long long>(static_cast<double>(md.u) * static_cast<double>(W));
    if (W == 0)
      Tu = 0;
    else if (Tu >= W)
      Tu = W - 1;
    // the first slice with kept mass whose running sum passes Tu (else the last
    // slice with kept mass, else slice 0)
    int st = wave_min(kt > 0 && inc > Tu ? lane : 64);
    if (st == 64) st = wave_max(kt > 0 ? lane : -1);
    unsigned long long rem = 0;
    if (st < 0) {
      st = 0;
    } else {
      rem = Tu - (rdl(inc, st) - rdl(kt, st));
    }
    if (lane == 0) {
      sh.sel[0] = st;
      sh.selu[0] = rem;
      sh.sel[1] = static_cast<int>(all_ties ? 0xffffffffu : sh.tcnt[st]);
    }
  }
  __syncthreads();
  const int st = sh.sel[0];
  const unsigned long long rem = sh.selu[0];
  const unsigned int tl = static_cast<unsigned int>(sh.sel[1]);
  __syncthreads();
  return walk<DT, EPT, VECOK>(a, r, st, Mp, rem, tau, tl, sh);
}

// ---- radix selection over the gathered candidates (LDS).  Over candidates
// with pred(c), values of the field F (the z' key, scanned in descending
// order, or the index, ascending) are scanned with measure 1 (counts) or the
// candidate's fixed-point mass; returns the first value v at which
// before + measure(v) >= target (> target when strict) with measure(v) > 0,
// where before is the measure of the values scanned before v.  When no value
// qualifies, the last value with a positive measure is returned.  *before_out
// gets `before`, *gcount the number of candidates equal to v.  8-bit digits;
// the leading bits all participants share are skipped.  Whole workgroup.
template <int DT, bool BY_KEY, bool MASSM, typename PRED>
__device__ __forceinline__ unsigned int cselect(int n, PRED pred, float Mp, unsigned long long target, bool strict, RLds& sh,
                                unsigned long long* before_out, unsigned int* gcount) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  (void)Mp;
  auto field = [](unsigned long long c) {
    return BY_KEY ? static_cast<unsigned int>(c) : static_cast<unsigned int>(c >> 32);
  };
  auto meas = [&](int c) -> unsigned long long { return MASSM ? sh.cmq[c] : 1ull; };
  unsigned int lo = 0xffffffffu, hi = 0u;
  for (int c = tid; c < n; c += THREADS) {
    const unsigned long long e = sh.cand[c];
    if (pred(e) && meas(c) > 0) {
      lo = min(lo, field(e));
      hi = max(hi, field(e));
    }
  }
  lo = wave_min(lo);
  hi = wave_max(hi);
  if (tid == 0) {
    sh.kmin = 0xffffffffu;
    sh.kmax = 0u;
  }
  __syncthreads();
  if (lane == 0) {
    atomicMin(&sh.kmin, lo);
    atomicMax(&sh.kmax, hi);
  }
  __syncthreads();
  lo = sh.kmin;
  hi = sh.kmax;
  __syncthreads();
  if (lo > hi) {  // no participant with a positive measure
    *before_out = 0;
    *gcount = 0;
    return 0;
  }
  int shift = 0;
  if (lo != hi) shift = ((31 - __clz(static_cast<int>(lo ^ hi))) >> 3) << 3;
  unsigned int mask = shift + 8 >= 32 ? 0u : ~((1u << (shift + 8)) - 1u);
  unsigned int prefix = lo & mask;
  unsigned long long before = 0;
  unsigned int g = 0;
  for (; shift >= 0; shift -= 8) {
    for (int d = tid; d < NB; d += THREADS) {
      sh.sl.hc[d] = 0u;
      sh.sl.hm[d] = 0ull;
    }
    __syncthreads();
    for (int c = tid; c < n; c += THREADS) {
      const unsigned long long e = sh.cand[c];
      const unsigned int f = field(e);
      if (pred(e) && (f & mask) == prefix) {
        const unsigned long long m = meas(c);
        if (m > 0) {
          const int d = static_cast<int>((f >> shift) & 255u);
          const int pos = BY_KEY ? NB - 1 - d : d;
          atomicAdd(&sh.sl.hc[pos], 1u);
          if (MASSM) atomicAdd(&sh.sl.hm[pos], m);
        }
      }
    }
    __syncthreads();
    if (wid == 0) {
      unsigned long long val[4];
      unsigned int cnt[4];
      unsigned long long sum = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        cnt[q] = sh.sl.hc[4 * lane + q];
        val[q] = MASSM ? sh.sl.hm[4 * lane + q] : static_cast<unsigned long long>(cnt[q]);
        sum += val[q];
      }
      const unsigned long long inc = wave_incl_scan_dpp(sum);
      unsigned long long run = before + inc - sum;
      int found = NB, lastne = -1;
      unsigned long long bef = 0, bef_last = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int pos = 4 * lane + q;
        if (found == NB && val[q] > 0 && (strict ? run + val[q] > target : run + val[q] >= target)) {
          found = pos;
          bef = run;
        }
        if (val[q] > 0) {
          lastne = pos;
          bef_last = run;
        }
        run += val[q];
      }
      int best = wave_min(found);
      unsigned long long b;
      if (best < NB) {
        b = rdl(bef, best >> 2);
      } else {
        best = wave_max(lastne);
        if (best < 0) best = 0;
        b = rdl(bef_last, best >> 2);
      }
      if (lane == 0) {
        sh.sel[2] = best;
        sh.sel[3] = static_cast<int>(sh.sl.hc[best]);
        sh.selu[1] = b;
      }
    }
    __syncthreads();
    const int pos = sh.sel[2];
    const unsigned int d = static_cast<unsigned int>(BY_KEY ? NB - 1 - pos : pos);
    prefix |= d << shift;
    mask |= 255u << shift;
    before = sh.selu[1];
    g = static_cast<unsigned int>(sh.sel[3]);
    __syncthreads();
  }
  *before_out = before;
  *gcount = g;
  return prefix;
}

// Block sum of the fixed-point masses of the candidates with pred.
template <int DT, typename PRED>
__device__ __forceinline__ unsigned long long cmass(int n, PRED pred, float Mp, RLds& sh) {
  (void)Mp;
  unsigned long long t = 0;
  for (int c = threadIdx.x; c < n; c += THREADS)
    if (pred(sh.cand[c])) t += sh.cmq[c];
  return block_sum<unsigned long long>(t, sh.sl.ru);
}

// Number of ties kept at a cutoff: the mass still to cover (need) in units of
// one tie's mass (wt), at least 1, at most g.
__device__ __forceinline__ unsigned int ties_kept(unsigned long long need, unsigned long long wt, unsigned int g) {
  unsigned long long t = g;
  // ceil(need / wt) when it is at most g: a double quotient (within one of
  // the integer one, the quotient being below 2^32) corrected by exact
  // products, in place of a 64-bit integer division
  if (wt > 0 && __umul64hi(g, wt) == 0ull && need < static_cast<unsigned long long>(g) * wt) {
    unsigned long long nd = static_cast<unsigned long long>(ceil(static_cast<double>(need) / static_cast<double>(wt)));
    if (nd > 0 && (nd - 1) * wt >= need) --nd;
    if (nd * wt < need) ++nd;
    t = nd;
  }
  if (t == 0) t = 1;
  return static_cast<unsigned int>(t);
}

// Publish wave 0's bracket [klo, khi] -> z-key bracket to the workgroup.
template <int DT>
__device__ __forceinline__ void set_bracket(Plan& pl, unsigned int klo, unsigned int khi, float Tr, RLds& sh) {
  // the z-key bracket [zlo, zhi] of the elements whose z' key lies in
  // [klo, khi]: its two ends, one wave each
  const int wid = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (wid == 0) {
    const unsigned int zl = gkey<DT>(kval<DT>(klo), Tr);
    if (lane == 0) sh.sel[6] = static_cast<int>(zl);
  } else if (wid == 1) {
    unsigned int zh = KEY_POS_INF;
    if (khi < key_hi<DT>()) {
      const unsigned int g = gkey<DT>(kval<DT>(khi + 1u), Tr);
      zh = g == 0u ? 0u : g - 1u;
    }
    if (lane == 0) sh.sel[7] = static_cast<int>(zh);
  }
  __syncthreads();
  pl.zlo = static_cast<unsigned int>(sh.sel[6]);
  pl.zhi = static_cast<unsigned int>(sh.sel[7]);
  __syncthreads();
}

// Digit level over the key range [klo, khi]: 256 bins of 2^sh keys from kb.
__device__ __forceinline__ void set_digits(Plan& pl, unsigned int klo, unsigned int khi) {
  pl.flags &= ~static_cast<unsigned int>(FL_VGRID);
  pl.kb = klo;
  const unsigned int span = khi - klo;
  const int bl = span ? 32 - __clz(static_cast<int>(span)) : 0;
  pl.sh = static_cast<unsigned int>(bl > 8 ? bl - 8 : 0);
}

// minp_key for the whole workgroup (wave 0 searches; uniform control flow).
template <int DT>
__device__ __forceinline__ unsigned int minp_key_block(float mr, float Mp, float nc, bool minf, RLds& sh) {
  if (threadIdx.x < 64) {
    const unsigned int t = minp_key<DT>(mr, Mp, nc, minf);
    if (threadIdx.x == 0) sh.sel[5] = static_cast<int>(t);
  }
  __syncthreads();
  const unsigned int t = static_cast<unsigned int>(sh.sel[5]);
  __syncthreads();
  return t;
}

// A row whose min_p keeps less than its top-k / top-p set keeps every z' key
// from tm: its per-slice kept masses are summed by a DRAWSUM pass.
template <int DT>
__device__ __forceinline__ void plan_minp_drawsum(Plan& pl, unsigned int tm, float Tr, RLds& sh) {
  pl.phase = PH_DRAWSUM;
  pl.fkey = tm;
  pl.target = 0;
  pl.cabove = 0u;
  set_bracket<DT>(pl, tm, key_hi<DT>(), Tr, sh);
}

// ---- the deciding step of a stage for row r (whole workgroup): reads the
// slices' results, then either writes the sampled id or leaves the next plan in
// sh.sl.pw and in the row's plan words.
template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ void finish_stage(const Args& a, int r, unsigned int ph, const unsigned long long* pwsrc,
                                             RLds& sh) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int S = a.S;
  // The slices' results for phase ph, requested together with the plan words
  // (pwsrc: the row's plan in global memory, or its copy in LDS): thread t owns
  // histogram bin t and sums every slice's cumulative count and mass at t;
  // thread t < S holds slice t's mass above the bracket so far, or its kept mass.
  const bool hist = ph == PH_COUNT || ph == PH_MASS;
  const bool mass = ph == PH_MASS;
  // (a gathering row's candidate slots are requested here too, in the same
  // memory round trip as its plan; unused slots hold stale words that are
  // never stored)
  unsigned long long cv[CAP / THREADS];
  if (ph == PH_GATHER) {
    const unsigned long long* src = a.cand + static_cast<size_t>(r) * CAP;
#pragma unroll
    for (int k = 0; k < CAP / THREADS; ++k) cv[k] = src[tid + k * THREADS];
  }
  const size_t o0 = static_cast<size_t>(r) * S * NB;
  unsigned int Cc = 0;
  unsigned long long Mc = 0;
  for (int t0 = 0; t0 < S; t0 += 32) {
    unsigned int cc[32];
    unsigned long long mc[32];
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const size_t o = o0 + static_cast<size_t>(t0 + j) * NB + tid;
      cc[j] = (hist && t0 + j < S) ? a.hcnt[o] : 0u;
      mc[j] = (mass && t0 + j < S) ? a.hmass[o] : 0ull;
    }
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      Cc += cc[j];
      Mc += mc[j];
    }
  }
  [[maybe_unused]] const int stamp_id = r;
  if (mass) MLXF_S1_STAMP(mlxf_m_stamps, 0);
  unsigned long long pre = 0;
  if (tid < S) {
    if (mass) pre = a.above[static_cast<size_t>(r) * S + tid];
    if (ph == PH_DRAWSUM) pre = a.dsum[static_cast<size_t>(r) * S + tid];
  }
  const unsigned int ng = (ph == PH_GATHER && tid == 0) ? a.ncand[r] : 0u;
  Plan pl = plan_unpack(pwsrc);
  const Mode md = decode<DT>(a, r);
  const float Mp = pl.Mp;
  const float nc = -(Mp * LOG2E);
  const bool minf = !__builtin_isfinite(Mp);
  const unsigned int khi_all = key_hi<DT>(), klo_all = key_lo<DT>();
  bool done = false;
  int id = 0;

  if (hist) {
    const unsigned long long abp = pre;
    const unsigned long long mcum = mass ? Mc : static_cast<unsigned long long>(Cc);
    sh.sl.hc[tid] = Cc;
    sh.sl.hm[tid] = mcum;
    if (tid == 0) sh.sel[4] = NB;
    __syncthreads();
    if (mass && pl.target == 0) {
      // first mass level: the nucleus target p * W over the participants
      const unsigned long long PW =
          static_cast<unsigned long long>(ceil(static_cast<double>(md.pr) * static_cast<double>(sh.sl.hm[NB - 1])));
      pl.target = PW < 1 ? 1 : PW;
    }
    // the chosen bin: the first whose cumulative measure reaches the target
    // (the total, should rounding leave the target out of reach)
    {
      const unsigned long long tgt = pl.target < sh.sl.hm[NB - 1] ? pl.target : sh.sl.hm[NB - 1];
      const unsigned long long bal = __ballot(mcum >= tgt);
      if (bal && lane == 0) atomicMin(&sh.sel[4], wid * 64 + __ffsll(static_cast<long long>(bal)) - 1);
    }
    __syncthreads();
    if (mass) MLXF_S1_STAMP(mlxf_m_stamps, 1);
    const int bstar = sh.sel[4] < NB ? sh.sel[4] : NB - 1;
    const unsigned long long abv = bstar > 0 ? sh.sl.hm[bstar - 1] : 0ull;  // measure above the bin
    const unsigned int cabv = bstar > 0 ? sh.sl.hc[bstar - 1] : 0u;         // participants above it
    const unsigned int cstar = sh.sl.hc[bstar] - cabv;                     // participants in it
    // per slice (thread t < S for slice t): the participants in the bin, and
    // the mass above it (MASS); the cumulative words around the bin are re-read
    // (they are in L2 by now)
    if (tid < S) {
      const size_t os = o0 + static_cast<size_t>(tid) * NB;
      const unsigned int cb = a.hcnt[os + bstar];
      const unsigned int cb1 = bstar > 0 ? a.hcnt[os + bstar - 1] : 0u;
      const unsigned long long mb1 = (mass && bstar > 0) ? a.hmass[os + bstar - 1] : 0ull;
      sh.tcnt[tid] = cb - cb1;
      if (mass) {
        sh.kept[tid] = abp + mb1;
        a.above[static_cast<size_t>(r) * S + tid] = abp + mb1;
      }
    }
    // key range [klo, khi] of the chosen bin: wave 0 the low edge, wave 1 the
    // high edge, wave 2 the first key with a positive mass
    if (mass) MLXF_S1_STAMP(mlxf_m_stamps, 2);
    if (tid == 0) {
      sh.sel[6] = 0;
      sh.sel[7] = static_cast<int>(khi_all);
      sh.sel[3] = static_cast<int>(klo_all);
    }
    __syncthreads();
    if (pl.flags & FL_VGRID) {
      auto vb = [&](unsigned int k) { return vbin_x(wlog2(kval<DT>(k), nc), pl.R2); };
      // (bin b's upper edge in z': vbin_x(x) <= b once x > -(b + 1) / R2, with
      // x = z' log2 e + nc: the search's guess)
      auto edge = [&](int b) {
        const float ze = (-static_cast<float>(b + 1) / pl.R2 - nc) * (1.0f / LOG2E);
        return __builtin_isfinite(ze) ? zkey<DT>(ze) : klo_all;
      };
      if (wid == 0) {
        const unsigned int klo =
            wave_search_near(klo_all, khi_all, edge(bstar), [&](unsigned int k) { return vb(k) <= bstar; });
        if (lane == 0) sh.sel[6] = static_cast<int>(klo);
      } else if (wid == 1 && bstar > 0) {
        const unsigned int nx =
            wave_search_near(klo_all, khi_all, edge(bstar - 1), [&](unsigned int k) { return vb(k) <= bstar - 1; });
        if (lane == 0) sh.sel[7] = static_cast<int>(nx > klo_all ? nx - 1u : klo_all);
      }
    } else if (tid == 0) {
      const unsigned long long lo64 =
          static_cast<unsigned long long>(pl.kb) + (static_cast<unsigned long long>(NB - 1 - bstar) << pl.sh);
      const unsigned long long hi64 = lo64 + (1ull << pl.sh) - 1ull;
      sh.sel[6] = static_cast<int>(lo64);
      sh.sel[7] = static_cast<int>(hi64 < khi_all ? hi64 : khi_all);
    }
    if (mass && wid == 2) {
      // elements whose mass quantises to zero never count: the bracket starts
      // at the first key with a positive mass
      // (a mass is positive from weight 2^-40 up: x >= -40)
      const float ze = (-40.0f - nc) * (1.0f / LOG2E);
      const unsigned int kq = wave_search_near(klo_all, khi_all, __builtin_isfinite(ze) ? zkey<DT>(ze) : klo_all,
                                               [&](unsigned int k) { return q40(wfun(kval<DT>(k), Mp, nc, minf)) > 0; });
      if (lane == 0) sh.sel[3] = static_cast<int>(kq);
    }
    __syncthreads();
    {
      unsigned int klo = static_cast<unsigned int>(sh.sel[6]), khi = static_cast<unsigned int>(sh.sel[7]);
      if (klo < pl.fkey) klo = pl.fkey;
      if (klo < static_cast<unsigned int>(sh.sel[3])) klo = static_cast<unsigned int>(sh.sel[3]);
      if (khi < klo) khi = klo;
      __syncthreads();
      if (tid == 0) {
        sh.sel[6] = static_cast<int>(klo);
        sh.sel[7] = static_cast<int>(khi);
      }
    }
    __syncthreads();
    if (mass) MLXF_S1_STAMP(mlxf_m_stamps, 3);
    const unsigned int klo = static_cast<unsigned int>(sh.sel[6]);
    const unsigned int khi = static_cast<unsigned int>(sh.sel[7]);
    __syncthreads();
    const bool exact = klo == khi;
    const unsigned long long rest = pl.target > abv ? pl.target - abv : 1ull;  // still to cover in the bin
    if (!mass) {
      const unsigned int nge = pl.cabove + cabv + cstar;  // participants with key >= klo
      if (nge <= CAP) {
        // gather everything from the bin's low edge up: the k-th largest, the
        // nucleus and the draw are then decided on the candidates
        pl.phase = PH_GATHER;
        pl.flags |= FL_GALL;
        set_bracket<DT>(pl, klo, khi_all, md.Tr, sh);
        pl.target = static_cast<unsigned long long>(md.kk);
      } else if (exact) {
        // the k-th largest z' is klo; every tie is kept
        pl.fkey = klo;
        pl.cabove = 0u;
        set_bracket<DT>(pl, klo, khi_all, md.Tr, sh);
        pl.target = 0;
        if (pl.flags & FL_TOPP) {
          pl.phase = PH_MASS;
          pl.flags &= ~static_cast<unsigned int>(FL_TOPP);
          plan_level1<DT>(pl, fminf(-wlog2(kval<DT>(klo), nc), MASS_LOG2_SPAN));
          for (int t = tid; t < S; t += THREADS) a.above[static_cast<size_t>(r) * S + t] = 0ull;
        } else {
          pl.phase = PH_DRAWSUM;
          if (md.mr > 0.0f) {
            const unsigned int tm = minp_key_block<DT>(md.mr, Mp, nc, minf, sh);
            if (tm > pl.fkey) pl.fkey = tm;
          }
        }
      } else {
        set_digits(pl, klo, khi);
        pl.cabove += cabv;
        pl.target = rest;
        set_bracket<DT>(pl, klo, khi, md.Tr, sh);
      }
    } else {
      const unsigned int tm = (exact && md.mr > 0.0f) ? minp_key_block<DT>(md.mr, Mp, nc, minf, sh) : 0u;
      if (exact && tm > klo) {
        plan_minp_drawsum<DT>(pl, tm, md.Tr, sh);
      } else if (exact) {
        // cutoff value klo: its first t ties (lowest indices) are kept
        const unsigned long long wt = q40(wfun(kval<DT>(klo), Mp, nc, minf));
        const unsigned int t = ties_kept(rest, wt, cstar);
        if (tid == 0) {
          unsigned int before = 0;
          for (int s2 = 0; s2 < S; ++s2) {
            const unsigned int c = sh.tcnt[s2];
            const unsigned int kt = t > before ? (t - before < c ? t - before : c) : 0u;
            before += c;
            sh.tcnt[s2] = kt;
            sh.kept[s2] += static_cast<unsigned long long>(kt) * wt;
          }
        }
        __syncthreads();
        id = draw<DT, EPT, VECOK>(a, r, md, Mp, klo, false, sh);
        done = true;
      } else if (cstar <= CAP) {
        pl.phase = PH_GATHER;
        pl.target = rest;
        set_bracket<DT>(pl, klo, khi, md.Tr, sh);
        MLXF_S1_STAMP(mlxf_m_stamps, 4);
      } else {
        set_digits(pl, klo, khi);
        pl.target = rest;
        set_bracket<DT>(pl, klo, khi, md.Tr, sh);
      }
    }
  } else if (ph == PH_DRAWSUM) {
    if (tid < S) sh.kept[tid] = pre;
    __syncthreads();
    id = draw<DT, EPT, VECOK>(a, r, md, Mp, pl.fkey, true, sh);
    done = true;
  } else if (ph == PH_GATHER) {
    [[maybe_unused]] const int stamp_id = r;
    MLXF_S1_STAMP(mlxf_d1_stamps, 8);
    if (tid == 0) {
      sh.ncand = ng < CAP ? ng : CAP;
      a.ncand[r] = 0u;
    }
    __syncthreads();
    const int n = static_cast<int>(sh.ncand);
#pragma unroll
    for (int k = 0; k < CAP / THREADS; ++k) {
      const int c = tid + k * THREADS;
      if (c < n) {
        sh.cand[c] = cv[k];
        sh.cmq[c] = q40(wfun(kval<DT>(static_cast<unsigned int>(cv[k])), Mp, nc, minf));
      }
    }
    __syncthreads();
    MLXF_S1_STAMP(mlxf_d1_stamps, 9);
    MLXF_S1_VAL(mlxf_d1_stamps, 14, n);
    unsigned long long bef;
    unsigned int g;
    if (pl.flags & FL_GALL) {
      // k-th largest z' (with multiplicity), then the nucleus inside the top k
      auto all = [](unsigned long long) { return true; };
      const unsigned int tk = cselect<DT, true, false>(n, all, Mp, pl.target, false, sh, &bef, &g);
      unsigned int tau = tk;
      unsigned int cut = 0xffffffffu;  // last kept index among the ties at tau
      if (pl.flags & FL_TOPP) {
        auto ink = [tk](unsigned long long e) { return static_cast<unsigned int>(e) >= tk; };
        const unsigned long long Wk = cmass<DT>(n, ink, Mp, sh);
        unsigned long long PW =
            static_cast<unsigned long long>(ceil(static_cast<double>(md.pr) * static_cast<double>(Wk)));
        if (PW < 1) PW = 1;
        unsigned long long pgt;
        tau = cselect<DT, true, true>(n, ink, Mp, PW, false, sh, &pgt, &g);
        const unsigned long long wt = q40(wfun(kval<DT>(tau), Mp, nc, minf));
        const unsigned int t = ties_kept(PW > pgt ? PW - pgt : 0ull, wt, g);
        if (t < g) {
          auto eq = [tau](unsigned long long e) { return static_cast<unsigned int>(e) == tau; };
          cut = cselect<DT, false, false>(n, eq, Mp, t, false, sh, &bef, &g);
        }
      }
      // min_p keeps z' keys from tm (every candidate at or above the bracket's
      // low edge is here, so it applies to them directly)
      const unsigned int tm = md.mr > 0.0f ? minp_key_block<DT>(md.mr, Mp, nc, minf, sh) : 0u;
      auto kept = [tau, cut, tm](unsigned long long e) {
        const unsigned int k = static_cast<unsigned int>(e);
        return k >= tm && (k > tau || (k == tau && static_cast<unsigned int>(e >> 32) <= cut));
      };
      const unsigned long long Wf = cmass<DT>(n, kept, Mp, sh);
      unsigned long long Tu = static_cast<unsigned long long>(static_cast<double>(md.u) * static_cast<double>(Wf));
      if (Wf == 0)
        Tu = 0;
      else if (Tu >= Wf)
        Tu = Wf - 1;
      id = static_cast<int>(cselect<DT, false, true>(n, kept, Mp, Tu, true, sh, &bef, &g));
      done = true;
    } else {
      // nucleus cutoff inside the bin: the remaining target over the candidates
      auto all = [](unsigned long long) { return true; };
      unsigned long long pgt;
      const unsigned int tau = cselect<DT, true, true>(n, all, Mp, pl.target, false, sh, &pgt, &g);
      MLXF_S1_STAMP(mlxf_d1_stamps, 10);
      const unsigned long long wt = q40(wfun(kval<DT>(tau), Mp, nc, minf));
      const unsigned int t = ties_kept(pl.target > pgt ? pl.target - pgt : 0ull, wt, g);
      unsigned int cut = 0xffffffffu;
      if (t < g) {
        auto eq = [tau](unsigned long long e) { return static_cast<unsigned int>(e) == tau; };
        cut = cselect<DT, false, false>(n, eq, Mp, t, false, sh, &bef, &g);
      }
      MLXF_S1_STAMP(mlxf_d1_stamps, 11);
      const unsigned int tm = md.mr > 0.0f ? minp_key_block<DT>(md.mr, Mp, nc, minf, sh) : 0u;
      if (tm > tau) {
        plan_minp_drawsum<DT>(pl, tm, md.Tr, sh);
      } else {
        // per-slice kept mass: above the bin, plus the kept candidates
        for (int t2 = tid; t2 < S; t2 += THREADS) {
          sh.kept[t2] = a.above[static_cast<size_t>(r) * S + t2];
          sh.tcnt[t2] = 0u;
        }
        __syncthreads();
        for (int c = tid; c < n; c += THREADS) {
          const unsigned long long e = sh.cand[c];
          const unsigned int k = static_cast<unsigned int>(e);
          const unsigned int i = static_cast<unsigned int>(e >> 32);
          // the slice length is THREADS * EPT, a power of two: a shift
          const int st = static_cast<int>(i / static_cast<unsigned int>(THREADS * EPT));
          if (k > tau || (k == tau && i <= cut)) {
            atomicAdd(&sh.kept[st], sh.cmq[c]);
            if (k == tau) atomicAdd(&sh.tcnt[st], 1u);
          }
        }
        __syncthreads();
        MLXF_S1_STAMP(mlxf_d1_stamps, 12);
        id = draw<DT, EPT, VECOK>(a, r, md, Mp, tau, false, sh);
        MLXF_S1_STAMP(mlxf_d1_stamps, 13);
        done = true;
      }
    }
  }
  if (done) pl.phase = PH_DONE;
  if (tid == 0) {
    if (done) write_out<DT>(a, r, id, pl.lse, md.want_lp);
    plan_store(a, r, pl);
    sh.sl.pw[RS_PHASE] = pack2(pl.phase, pl.flags);
    sh.sl.pw[RS_ZB] = pack2(pl.zlo, pl.zhi);
    sh.sl.pw[RS_DIG] = pack2(pl.kb, pl.sh);
    sh.sl.pw[RS_AUX] = pack2(pl.cabove, pl.fkey);
    sh.sl.pw[RS_GRID] = pack2(__float_as_uint(pl.Mp), __float_as_uint(pl.R2));
    sh.sl.pw[RS_TGT] = pl.target;
    sh.sl.pw[RS_LSE] = static_cast<unsigned long long>(__double_as_longlong(pl.lse));
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
}

// Refine stage `stage` (0-based), one workgroup per slice of each row on the
// stage's list.  The list and the plans come from the previous kernel.
template <int DT, int EPT, bool VECOK>
__global__ __launch_bounds__(THREADS) void k_scan(Args a, int stage) {
  __shared__ SLds sh;
  const int bid = static_cast<int>(blockIdx.x);
  const int S = a.S;
  const unsigned int n = a.actcnt[stage];
  const unsigned int e = a.actlist[static_cast<size_t>(stage) * a.B + bid / S];
  if (static_cast<unsigned int>(bid) >= n * static_cast<unsigned int>(S)) return;
  const int r = static_cast<int>(e & 0xffffu);
  const Plan pl = plan_unpack(a.rowst + static_cast<size_t>(r) * RS_WORDS);
  slice_stage<DT, EPT, VECOK>(a, r, bid % S, pl, sh);
}

// Finish row r here: run the remaining levels over the row's slices in this
// workgroup (the row plan is in sh.sl.pw).  Each level narrows the bracket or
// advances the phase: a selection takes a value-grid level and at most four
// 8-bit key-digit levels (a digit level whose bin is one key is exact), and
// the phases only move forward (COUNT, MASS, GATHER / DRAWSUM), so a row needs
// far fewer than SERIAL_MAX levels.  Should the bound ever be reached, the row
// still gets a defined id: its argmax.
template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ void serial_finish(const Args& a, int r, RLds& sh) {
  for (int it = 0; it < SERIAL_MAX && static_cast<unsigned int>(sh.sl.pw[RS_PHASE]) != PH_DONE; ++it) {
    const Plan pl = plan_unpack(sh.sl.pw);
    for (int s2 = 0; s2 < a.S; ++s2) {
      slice_stage<DT, EPT, VECOK>(a, r, s2, pl, sh.sl);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
    }
    // the slice passes' stores are complete; drop stale L1 lines before the
    // plain loads of the deciding step
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
    finish_stage<DT, EPT, VECOK>(a, r, pl.phase, sh.sl.pw, sh);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  }
  if (static_cast<unsigned int>(sh.sl.pw[RS_PHASE]) != PH_DONE && threadIdx.x == 0) {
    float bm = -INFINITY;
    int bi = 0;
    for (int s2 = 0; s2 < a.S; ++s2) {
      const unsigned long long w0 = a.rec[(static_cast<size_t>(r) * a.S + s2) * REC];
      const float m = __uint_as_float(static_cast<unsigned int>(w0));
      if (m > bm) {
        bm = m;
        bi = static_cast<int>(w0 >> 32);
      }
    }
    const Plan pl = plan_unpack(sh.sl.pw);
    write_out<DT>(a, r, bi, pl.lse, decode<DT>(a, r).want_lp);
  }
}

// Refine stage `stage`, one workgroup per row on the stage's list: decide, and
// put the row on the next stage's list if it is still open.  The last stage
// launched finishes every row itself.
template <int DT, int EPT, bool VECOK>
__global__ __launch_bounds__(THREADS, 1) void k_decide(Args a, int stage, int last) {
  __shared__ RLds sh;
  const int tid = threadIdx.x;
  const int bid = static_cast<int>(blockIdx.x);
  const unsigned int n = a.actcnt[stage];
  const unsigned int e = a.actlist[static_cast<size_t>(stage) * a.B + bid];
  if (static_cast<unsigned int>(bid) >= n) return;
  const int r = static_cast<int>(e & 0xffffu);
  [[maybe_unused]] const int stamp_id = r;
  MLXF_S1_STAMP(mlxf_d1_stamps, 7);
  finish_stage<DT, EPT, VECOK>(a, r, e >> 16, a.rowst + static_cast<size_t>(r) * RS_WORDS, sh);
  MLXF_S1_STAMP(mlxf_d1_stamps, 15);
  if (static_cast<unsigned int>(sh.sl.pw[RS_PHASE]) == PH_DONE) return;
  if (!last) {
    if (tid == 0) enlist(a, stage + 1, r, static_cast<unsigned int>(sh.sl.pw[RS_PHASE]));
    return;
  }
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  serial_finish<DT, EPT, VECOK>(a, r, sh);
}

// Shared memory of k_decide1: the list stage, then (when no refine stage is
// launched) the refine state of a row finished here.
union D1Shared {
  D1Lds d;
  RLds r;
};

// Row r after its slices' first pass (whole workgroup): argmax, log-sum-exp,
// top_logprobs, top-k <= 63, and a plan for every other sampling row, which
// goes on the first refine stage's list (nstage > 0) or is finished here.
template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ void decide1_row(const Args& a, int r, int nstage, D1Shared& shu) {
  D1Lds& sh = shu.d;
  [[maybe_unused]] const int stamp_id = r;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int S = a.S;
  // candidate slots: wave w takes slices w, w + 4, w + 8, ... (lane l their
  // slots l and l + 64).  Those of the first 32 slices are requested before
  // the row's parameters say whether they are needed: one memory round trip
  // for the records, the parameters and (up to 32 slices) every candidate.
  constexpr int SPW = 8;  // slices per wave and round
  const unsigned long long* src = a.list + static_cast<size_t>(r) * S * SCAP;
  unsigned long long cw[2 * SPW];
  auto load_round = [&](int base) {
#pragma unroll
    for (int m = 0; m < SPW; ++m) {
      const int s2 = base + wid + WAVES * m;
#pragma unroll
      for (int h = 0; h < 2; ++h) cw[2 * m + h] = s2 < S ? src[s2 * SCAP + h * 64 + lane] : 0ull;
    }
  };
  load_round(0);
  const Mode md = decode<DT>(a, r);
  MLXF_S1_STAMP(mlxf_d1_stamps, 0);
  const int SP = (S + 3) & ~3;  // row stride of the threshold table (zero padded)
  if (tid < SP) {
    // (all seven words in one request: those of the list are not written for
    // rows without one, and are then unused)
    const bool real = tid < S;
    const unsigned long long* rp = a.rec + (static_cast<size_t>(r) * S + (real ? tid : 0)) * REC;
    const unsigned long long w0 = rp[0], w1 = rp[1], w2 = rp[2], w3 = rp[3], w4 = rp[4], w5 = rp[5], w6 = rp[6],
                             w7 = rp[7];
    if (real) {
      sh.szmax[tid] = __uint_as_float(static_cast<unsigned int>(w0));
      sh.szarg[tid] = static_cast<int>(w0 >> 32);
      sh.szmin[tid] = __uint_as_float(static_cast<unsigned int>(w1));
      sh.slse[tid] = __longlong_as_double(static_cast<long long>(w2));
      sh.sn[tid] = static_cast<int>(w5 >> 32);
      sh.swsum[tid] = __longlong_as_double(static_cast<long long>(w7));
    }
    if (md.need_list) {
      const unsigned int t[7] = {static_cast<unsigned int>(w3), static_cast<unsigned int>(w3 >> 32),
                                 static_cast<unsigned int>(w4), static_cast<unsigned int>(w4 >> 32),
                                 static_cast<unsigned int>(w5), static_cast<unsigned int>(w6),
                                 static_cast<unsigned int>(w6 >> 32)};
#pragma unroll
      for (int j = 0; j < 7; ++j) sh.thr[j * SP + tid] = real ? t[j] : 0u;
    }
  }
  if (tid == 0) sh.ncnt = 0;
  __syncthreads();
  MLXF_S1_STAMP(mlxf_d1_stamps, 1);
  // the row's max, lowest argmax, minimum and log-sum-exp from the slice
  // records, by one wave (the last, when it has nothing else to do)
  auto row_stats = [&]() {
    const float zm = lane < S ? sh.szmax[lane] : -INFINITY;
    const int za = lane < S ? sh.szarg[lane] : INT_MAX;
    float rm = zm;
    int ra = za;
    wave_best(rm, ra);
    double part = (lane < S && md.need_lse) ? sh.slse[lane] * wexp_d(zm, rm) : 0.0;
    part = wave_sum(part);
    const float mn = wave_min(lane < S ? sh.szmin[lane] : INFINITY);
    if (lane == 0) {
      sh.zmax = rm;
      sh.zarg = ra;
      sh.zmin = mn;
      sh.lse = md.need_lse ? static_cast<double>(rm) + log(part) : static_cast<double>(NAN);
    }
    if (md.kind == KIND_TOPP && md.need_list) {
      // Bounds on W = sum floor(2^40 w_i), w_i = exp2(RN(z'_i log2 e + nc)),
      // nc = -RN(Mp log2 e), from the slice sums of w'_i = exp2(RN(z'_i log2 e
      // + ncs)) (ncs: the same with the slice's own max): z'_i log2 e + nc is
      // (z'_i log2 e + ncs) + (nc - ncs) exactly, so for every element of
      // weight >= 2^-41 (both arguments in [-41, 0]) the two roundings and the
      // two exp2 evaluations (each within 2^-22) put w_i within 2^-17.9 of
      // w'_i 2^(nc - ncs) relatively; an element below 2^-41 has floor 0 and
      // adds under half a unit to the float sum; floor loses under one unit
      // per element; the 32-term fp32 sums add at most 2^-19.  So W lies in
      // [Wf (1 - 2^-15) - 2V - 64, Wf (1 + 2^-15) + V + 64] with margin.
      // (No bound for an infinite, huge or tiny-temperature max.)
      const float Mp = zdiv<DT>(rm, md.Tr, md.y, false);
      const float nc = -(Mp * LOG2E);
      bool bad = !__builtin_isfinite(Mp) || fabsf(Mp) > 0x1p20f || md.tslow != 0;
      double wp = 0.0;
      if (lane < S && !bad) {
        const double ws = sh.swsum[lane];
        const float ncs = -(zdiv<DT>(sh.szmax[lane], md.Tr, md.y, true) * LOG2E);
        if (!(ws >= 0.0)) {
          bad = true;
        } else if (ws > 0.0) {
          wp = ws * exp2(static_cast<double>(nc) - static_cast<double>(ncs));
        }
      }
      const bool anybad = __ballot(bad) != 0ull;
      const double wf = wave_sum(wp) * 0x1p40;
      if (lane == 0) {
        const double slack = static_cast<double>(a.V) + 64.0;
        sh.wlo = wf * (1.0 - 0x1p-15) - 2.0 * slack;
        sh.whi = wf * (1.0 + 0x1p-15) + slack;
        sh.wok = (!anybad && __builtin_isfinite(wf)) ? 1 : 0;
      }
    }
  };
  if (md.need_list) {
    // theta, a key the row's 64th best reaches.  Slice s has at least j
    // elements at or above t_j(s), hence at least
    //   n_s(c) = 32 [t_64 >= c] + 16 [t_32 >= c] + 8 [t_16 >= c] + 4 [t_8 >= c]
    //          + 2 [t_4 >= c] + [t_2 >= c] + [t_1 >= c]
    // at or above c (the t_j decrease with j); theta is the largest of the 7S
    // keys t_j(s) with sum_s n_s(theta) >= 64, one thread per key.  An entry
    // of the row's best 64 is among its slice's candidates, so the candidates
    // at or above theta hold the row's best 64.
    auto okey = [](unsigned long long ent) {  // the value part of order_key
      const float v = __uint_as_float(static_cast<unsigned int>(ent));
      return f2key(v == 0.0f ? 0.0f : v);
    };
    // F(c) = sum_s n_s(c) over slices [s4b, s4e) x 4 (the seven levels' reads
    // in flight together)
    auto fcount = [&](unsigned int c, int s4b, int s4e) {
      int cnt[7] = {0, 0, 0, 0, 0, 0, 0};
      for (int s4 = s4b; s4 < s4e; ++s4) {
        uint4 t4[7];
#pragma unroll
        for (int j = 0; j < 7; ++j) t4[j] = reinterpret_cast<const uint4*>(&sh.thr[j * SP])[s4];
#pragma unroll
        for (int j = 0; j < 7; ++j)
          cnt[j] += (t4[j].x >= c ? 1 : 0) + (t4[j].y >= c ? 1 : 0) + (t4[j].z >= c ? 1 : 0) + (t4[j].w >= c ? 1 : 0);
      }
      return 32 * cnt[0] + 16 * cnt[1] + 8 * cnt[2] + 4 * cnt[3] + 2 * cnt[4] + cnt[5] + cnt[6];
    };
    unsigned int best = 0u;
    for (int q = tid; q < 7 * SP; q += THREADS) {
      const unsigned int c = sh.thr[q];
      if (fcount(c, 0, SP / 4) >= 64) best = max(best, c);
    }
    best = wave_max(best);
    if (lane == 0) sh.thw[wid] = best;
    if (wid == WAVES - 1) row_stats();
    __syncthreads();
    // (a key k of -0 passes the candidates of +0 and -0 alike: okey gives both
    // +0's key.  The float compare against thf is the same test: -0 == +0, and
    // a theta at or below -inf's key passes every candidate.)
    const unsigned int thk = max(max(sh.thw[0], sh.thw[1]), max(sh.thw[2], sh.thw[3]));
    const float thf = thk <= KEY_NEG_INF ? -INFINITY : key2f(thk);
    MLXF_S1_STAMP(mlxf_d1_stamps, 2);
    // the candidates at or above theta, as order keys, gathered into sv: per
    // wave and round the slices' ballots, then one LDS atomic for the wave's
    // places (the order of the waves varies from run to run; every reader
    // orders by key)
    auto lane_below = [&](unsigned long long b) {
      return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<unsigned int>(b >> 32),
                                                        __builtin_amdgcn_mbcnt_lo(static_cast<unsigned int>(b), 0u)));
    };
    for (int base = 0; base < S; base += WAVES * SPW) {
      if (base > 0) load_round(base);
      unsigned long long bal[2 * SPW];
      int tot = 0;
#pragma unroll
      for (int m = 0; m < SPW; ++m) {
        const int s2 = base + wid + WAVES * m;
        const int n2 = s2 < S ? sh.sn[s2] : 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const bool ok = (lane + 64 * h < n2) & (__uint_as_float(static_cast<unsigned int>(cw[2 * m + h])) >= thf);
          bal[2 * m + h] = __builtin_amdgcn_ballot_w64(ok);
          tot += static_cast<int>(__builtin_popcountll(bal[2 * m + h]));
        }
      }
      int wb = 0;
      if (lane == 0 && tot) wb = __hip_atomic_fetch_add(&sh.ncnt, tot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      wb = __builtin_amdgcn_readlane(wb, 0);
#pragma unroll
      for (int q = 0; q < 2 * SPW; ++q) {
        if (bal[q] == 0ull) continue;  // (uniform: most slot groups hold no candidate)
        const int p = wb + lane_below(bal[q]);
        if (((bal[q] >> lane) & 1ull) && p < CBUF) sh.sv[p] = order_key(cw[q]);
        wb += static_cast<int>(__builtin_popcountll(bal[q]));
      }
    }
    __syncthreads();
    const int nsv = sh.ncnt;
    MLXF_S1_STAMP(mlxf_d1_stamps, 3);
    MLXF_S1_VAL(mlxf_d1_stamps, 15, nsv);
    if (nsv <= THREADS) {
      // (the usual case) each candidate's place in the order is the number of
      // candidates with a larger key, counted over the list in LDS (read two
      // at a time, the same address in every lane) by P neighbouring lanes, a
      // share each; the best 64 go straight to their places
      int lp2 = 0;
      while (lp2 < 3 && (nsv << (lp2 + 1)) <= THREADS) ++lp2;
      const int P = 1 << lp2;
      const int c = tid >> lp2, part = tid & (P - 1);
      const int npair = nsv >> 1, per = (npair + P - 1) >> lp2;
      const unsigned long long mk = c < nsv ? sh.sv[c] : ~0ull;
      const ulonglong2* p2 = reinterpret_cast<const ulonglong2*>(sh.sv);
      int c4[4] = {0, 0, 0, 0};  // independent counts: no chain through one register
      int j = part * per;
      const int jend = min(npair, j + per);
      for (; j + 8 <= jend; j += 8) {  // eight reads in flight
        ulonglong2 q[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) q[u] = p2[j + u];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          c4[u & 3] += q[u].x > mk ? 1 : 0;
          c4[(u + 2) & 3] += q[u].y > mk ? 1 : 0;
        }
      }
      for (; j < jend; ++j) {
        const ulonglong2 q = p2[j];
        c4[0] += q.x > mk ? 1 : 0;
        c4[1] += q.y > mk ? 1 : 0;
      }
      if ((nsv & 1) && part == 0) c4[2] += sh.sv[nsv - 1] > mk ? 1 : 0;
      int rk = (c4[0] + c4[1]) + (c4[2] + c4[3]);
      if (P > 1) rk += xshf<1>(rk);  // the P shares (whole wave active)
      if (P > 2) rk += xshf<2>(rk);
      if (P > 4) rk += xshf<4>(rk);
      if (c < nsv && part == 0 && rk < LIST) {
        sh.mlist[rk].v = order_key_v(mk);
        sh.mlist[rk].i = order_key_i(mk);
      }
      if (tid >= nsv && tid < LIST) {
        sh.mlist[tid].v = -INFINITY;
        sh.mlist[tid].i = INT_MAX;
      }
    } else {
      // (many candidates) 64-entry chunks sorted by the waves and merged:
      // from LDS when they fit, else every slot from memory
      float lv = -INFINITY;
      int li = INT_MAX;
      if (nsv <= CBUF) {
        const int nch = (nsv + LIST - 1) / LIST;
        for (int ch = wid; ch < nch; ch += WAVES) {
          const int c = ch * LIST + lane;
          float cv = -INFINITY;
          int ci = INT_MAX;
          if (c < nsv) {
            const unsigned long long k = sh.sv[c];
            cv = order_key_v(k);
            ci = order_key_i(k);
          }
          wave_sort(cv, ci);
          wave_list_merge(lv, li, cv, ci);
        }
      } else {
        const int nch = S * SCAP / LIST;
        for (int ch = wid; ch < nch; ch += WAVES) {
          const int i = ch * LIST + lane;
          const unsigned long long w = src[i];
          const float v = __uint_as_float(static_cast<unsigned int>(w));
          const bool ok = (i & (SCAP - 1)) < sh.sn[i >> SCAP_LOG2] && okey(w) >= thk;
          float cv = ok ? v : -INFINITY;
          int ci = ok ? static_cast<int>(w >> 32) : INT_MAX;
          wave_sort(cv, ci);
          wave_list_merge(lv, li, cv, ci);
        }
      }
      tree_merge(lv, li, sh.lists, WAVES);
      if (wid == 0) {
        sh.mlist[lane].v = lv;
        sh.mlist[lane].i = li;
      }
    }
  } else if (wid == WAVES - 1) {
    row_stats();
  }
  __syncthreads();
  MLXF_S1_STAMP(mlxf_d1_stamps, 4);
  const double lse = sh.lse;
  if (a.K_max > 0 && tid < a.K_max) {  // top_logprobs: the first K of the best 64
    const size_t o = static_cast<size_t>(r) * a.K_max + tid;
    if (tid < md.K) {
      a.out_top_ids[o] = sh.mlist[tid].i;
      a.out_top_lp[o] = static_cast<float>(static_cast<double>(sh.mlist[tid].v) - lse);
    } else {
      a.out_top_ids[o] = -1;
      a.out_top_lp[o] = -INFINITY;
    }
  }
  Plan pl;
  pl.phase = PH_DONE;
  pl.flags = 0u;
  pl.zlo = KEY_NEG_INF;
  pl.zhi = KEY_POS_INF;
  pl.kb = 0u;
  pl.sh = 0u;
  pl.cabove = 0u;
  pl.fkey = key_lo<DT>();
  pl.Mp = 0.0f;
  pl.R2 = 0.0f;
  pl.target = 0ull;
  pl.lse = lse;
  if (!md.sampling) {
    if (tid == 0) write_out<DT>(a, r, sh.zarg, lse, md.want_lp);
    return;
  }
  const float M = sh.zmax;
  const float Mp = zdiv<DT>(M, md.Tr, md.y, false);  // max z' = z'(max z)
  pl.Mp = Mp;
  if (M == -INFINITY || (md.topp && !(md.pr > 0.0f))) {
    // nothing left to draw (every logit -inf, or a top-p that rounds to 0):
    // the reference's categorical is the argmax of the logits plus Gumbel
    // noise, -inf everywhere, whose first index is 0
    if (tid == 0) write_out<DT>(a, r, 0, lse, md.want_lp);
    return;
  }
  // A top-p row with a best-64 list (it wants top_logprobs) whose nucleus
  // provably ends inside the list is finished from it like a top-k row: with W (the row's total mass)
  // known only within [wlo, whi], the cut (keep while the mass before an entry
  // is below ceil(p W)) is taken at both ends; when both keep the same K < 64
  // entries and no element outside the list ties or passes the K-th z', that
  // is the cut for the exact W.  Otherwise the row goes on to the refine
  // stages.
  const bool plist = md.kind == KIND_TOPP && md.need_list && sh.wok != 0;
  if (md.kind == KIND_KLIST || plist) {
    // klist_resolve on two waves: wave 0 makes the cut (the kept entries are
    // a prefix of the (z' desc, index asc) order: top-k, then top-p while the
    // mass before an entry is < p W_k, then min_p, non-increasing weights),
    // while wave 1 sorts the list by index for the draw, each entry carrying
    // its place in that order (in the low 6 bits of 64 w, exact in a double)
    if (wid < 2) {
      float sv, wv;
      int si;
      double w;
      bool ok;
      float last_zp = 0.0f;
      int last_i = INT_MAX;
      if (plist) {
        plist_prep<DT>(md, Mp, sh.mlist, sv, si, wv, w, last_zp, last_i);
        ok = true;
      } else {
        ok = klist_prep<DT>(md, Mp, sh.mlist, sv, si, wv, w);
      }
      if (wid == 0) {
        if (ok) {
          const double incl = wave_incl_scan_dpp(w);
          const double Wk = rdl(incl, 63);
          bool keep = si != INT_MAX;
          if (plist) {
            const double pwl = fmax(ceil(static_cast<double>(md.pr) * sh.wlo), 1.0);
            const double pwh = fmax(ceil(static_cast<double>(md.pr) * sh.whi), 1.0);
            const bool kl = keep && (incl - w) < pwl, kh = keep && (incl - w) < pwh;
            const int nl = static_cast<int>(__builtin_popcountll(__ballot(kl)));
            const int nh = static_cast<int>(__builtin_popcountll(__ballot(kh)));
            const float zk = rdl(sv, nh > 0 ? nh - 1 : 0);
            ok = nl == nh && nh > 0 && nh < LIST && (last_i == INT_MAX || last_zp < zk);
            keep = kl;
          } else if (md.topp) {
            keep = keep && (incl - w) < ceil(static_cast<double>(md.pr) * Wk);
          }
          if (md.mr > 0.0f) {
            const float nc = -(Mp * LOG2E);
            keep = keep && wv >= minp_thr(md.mr, Mp, nc, !__builtin_isfinite(Mp));
          }
          const double Wf = wave_sum(keep ? w : 0.0);
          unsigned long long Tu = static_cast<unsigned long long>(static_cast<double>(md.u) * Wf);
          if (Wf == 0.0)
            Tu = 0;
          else if (static_cast<double>(Tu) >= Wf)
            Tu = static_cast<unsigned long long>(Wf) - 1;
          const int nk = static_cast<int>(__builtin_popcountll(__builtin_amdgcn_ballot_w64(keep)));
          if (lane == 0) {
            sh.kl_tu = Tu;
            sh.kl_nk = Wf == 0.0 ? -nk : nk;  // (negative: every kept weight is 0)
            sh.sel[1] = si;                   // (the draw's answer when nothing is kept)
          }
        }
        if (lane == 0) sh.sel[0] = ok ? 1 : 0;
        __syncthreads();
      } else {
        int ki = si;
        double kwp = ok ? w * 64.0 + static_cast<double>(lane) : 0.0;
        if (ok) wave_sort_idx(ki, kwp);
        __syncthreads();
        if (ok) {
          const int nkr = sh.kl_nk, nk = nkr < 0 ? -nkr : nkr;
          const unsigned long long kq = static_cast<unsigned long long>(kwp);
          const bool kept = ki != INT_MAX && static_cast<int>(kq & 63u) < nk;
          const double kw = kept ? static_cast<double>(kq >> 6) : 0.0;
          const double cum = wave_incl_scan_dpp(kw);
          const bool hit = kept && (nkr < 0 || (kw > 0.0 && cum > static_cast<double>(sh.kl_tu)));
          const int cand = wave_min(hit ? ki : INT_MAX);
          if (lane == 0 && cand != INT_MAX) sh.sel[1] = cand;
        }
      }
    } else {
      __syncthreads();
    }
    __syncthreads();
    MLXF_S1_STAMP(mlxf_d1_stamps, 5);
    if (sh.sel[0]) {
      if (tid == 0) write_out<DT>(a, r, sh.sel[1], lse, md.want_lp);
      MLXF_S1_STAMP(mlxf_d1_stamps, 6);
      return;
    }
  }
  const float nc = -(Mp * LOG2E);
  // full span of the row in log2 units (unknown, i.e. infinite, when the scan
  // did not take the minimum)
  const float spanc = sh.zmin == INFINITY ? INFINITY : -wlog2(zdiv<DT>(sh.zmin, md.Tr, md.y, false), nc);
  if (md.kind == KIND_KLIST || md.kind == KIND_KHIST) {
    pl.phase = PH_COUNT;
    pl.target = static_cast<unsigned long long>(md.kk);
    if (md.topp) pl.flags |= FL_TOPP;
    plan_level1<DT>(pl, spanc);
  } else if (md.kind == KIND_TOPP) {
    pl.phase = PH_MASS;
    plan_level1<DT>(pl, fminf(spanc, MASS_LOG2_SPAN));
    for (int t = tid; t < S; t += THREADS) a.above[static_cast<size_t>(r) * S + t] = 0ull;
  } else {
    pl.phase = PH_DRAWSUM;
    if (md.mr > 0.0f) {
      // min_p: the kept set is every z' key from tm
      if (wid == 0) {
        const unsigned int tm = minp_key<DT>(md.mr, Mp, nc, !__builtin_isfinite(Mp));
        if (lane == 0) sh.sel[2] = static_cast<int>(tm);
      }
      __syncthreads();
      pl.fkey = static_cast<unsigned int>(sh.sel[2]);
    }
  }
  if (tid == 0) plan_store(a, r, pl);
  if (nstage > 0) {
    if (tid == 0) enlist(a, 0, r, pl.phase);
    return;
  }
  // no refine stage is launched (the caller's parameters promised top-k <= 63
  // or greedy rows only): finish the row here
  __syncthreads();
  if (tid == 0) {
    shu.r.sl.pw[RS_PHASE] = pack2(pl.phase, pl.flags);
    shu.r.sl.pw[RS_ZB] = pack2(pl.zlo, pl.zhi);
    shu.r.sl.pw[RS_DIG] = pack2(pl.kb, pl.sh);
    shu.r.sl.pw[RS_AUX] = pack2(pl.cabove, pl.fkey);
    shu.r.sl.pw[RS_GRID] = pack2(__float_as_uint(pl.Mp), __float_as_uint(pl.R2));
    shu.r.sl.pw[RS_TGT] = pl.target;
    shu.r.sl.pw[RS_LSE] = static_cast<unsigned long long>(__double_as_longlong(pl.lse));
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  serial_finish<DT, EPT, VECOK>(a, r, shu.r);
}

template <int DT, int EPT, bool VECOK>
__global__ __launch_bounds__(THREADS, 1) void k_decide1(Args a, int nstage) {
  __shared__ D1Shared shu;
  decide1_row<DT, EPT, VECOK>(a, static_cast<int>(blockIdx.x), nstage, shu);
}

// LDS of the row-histogram path's fallback (the per-slice path over one row,
// first pass and deciding step in one workgroup, every refine level there).
union FbShared {
  S1Lds s1;
  D1Shared d1;
};

// ================================================================ host side ==

// Stage 0 (scan, decide), then `nst` refine stages (scan, decide); the last
// deciding kernel launched finishes every row still open.  nst < 0: the first
// scan only.
template <int DT, int EPT, bool VECOK>
hipError_t launch_ept(const Args& a, int nst, hipStream_t st) {
  const dim3 slices(static_cast<unsigned int>(a.B * a.S)), rows(static_cast<unsigned int>(a.B));
  hipLaunchKernelGGL((k_scan1<DT, EPT, VECOK>), slices, dim3(THREADS), 0, st, a);
  if (nst < 0) return hipGetLastError();  // the first pass alone (profiling)
  hipLaunchKernelGGL((k_decide1<DT, EPT, VECOK>), rows, dim3(THREADS), 0, st, a, nst);
  for (int i = 0; i < nst; ++i) {
    hipLaunchKernelGGL((k_scan<DT, EPT, VECOK>), slices, dim3(THREADS), 0, st, a, i);
    hipLaunchKernelGGL((k_decide<DT, EPT, VECOK>), rows, dim3(THREADS), 0, st, a, i, i == nst - 1 ? 1 : 0);
  }
  return hipGetLastError();
}

template <int DT>
hipError_t launch_dt(const Args& a, int ept, bool vecok, int nst, hipStream_t st) {
  switch (ept) {
    case 8:
      return vecok ? launch_ept<DT, 8, true>(a, nst, st) : launch_ept<DT, 8, false>(a, nst, st);
    case 16:
      return vecok ? launch_ept<DT, 16, true>(a, nst, st) : launch_ept<DT, 16, false>(a, nst, st);
    default:
      return vecok ? launch_ept<DT, 32, true>(a, nst, st) : launch_ept<DT, 32, false>(a, nst, st);
  }
}

}  // namespace
}  // namespace mlxf

#include "rowhist.hpp"
