// sampler.hip -- MI355X (gfx950) batched token sampler behind the C ABI in
// include/mlxf_sampler.h.
//
// Replaces the per-row MLX graph of Sampler::sample (src/sample/sampler.cpp:
// 141-166), run once per row by Worker::sample_rows (src/runtime/worker.cpp:
// 448-486), with ONE kernel launch over all rows of a [B, V] logits matrix.
//
// Grid (S, B): row r is cut into S slices of L = 256 * EPT elements (EPT up to
// 32); slice s is one 256-thread workgroup (4 waves, up to 256 VGPRs each, two
// workgroups per CU) that loads its whole slice into registers with 16-byte
// loads (one HBM read of the logits) and reduces it there:
//   * max and lowest-index argmax of z, and sum exp(z - max) when a logprob is
//     wanted;
//   * when top_logprobs or a top-k <= 63 is asked for: the slice's best 64
//     entries by (z desc, index asc).  The 64th best of the 256 per-thread
//     maxima bounds the slice's 64th best from below; the at most 64 * EPT
//     elements at or above it are sorted in 64-entry chunks and merged;
//   * top-k > 63: a 4096-bin count histogram of z keys gives the bin of the
//     slice's k-th largest z; everything from the (temperature-mapped) lower
//     edge of that bin up is written out as a candidate;
//   * temperature-only and top-p rows: the sum of w = exp(z' - max z') over the
//     slice (z' = z / T in the logits dtype), and for top-p a 2048-bin
//     histogram of z' keys with (count, truncated w) packed in one 64-bit word.
// The slice then takes a ticket on the row's counter; the workgroup that draws
// the row's last ticket finishes the row.  No workgroup ever waits for another.
//   * greedy: argmax, logprob and top_logprobs from the slice summaries;
//   * top-k <= 63: the merged best-64 list of the row decides everything in one
//     wave (the k-th largest z', the nucleus prefix, the draw), after checking
//     that the list holds every element at or above the k-th value of z';
//   * top-k > 63: 8-bit radix selections over the candidates;
//   * temperature-only: the slice that holds u * sum(w), then a walk of that
//     slice in vocabulary order;
//   * top-p: the combined histogram, with the bound of its truncation error,
//     brackets the nucleus boundary in a range R of bins; a compare-only pass
//     over the row collects R's elements and the exact mass of the smaller
//     side of R; radix selections over R's elements give the cutoff value and
//     the last kept index among its ties; then the walk of the one slice that
//     holds the draw.
// Masses that decide a cutoff are exact 64-bit fixed-point sums (2^-42 units)
// or fp64 sums in a fixed order, so every result is reproducible bit for bit.
// Data one workgroup leaves for another travels through device-coherent (sc1)
// loads and stores, so no L2-wide write-back is ever needed.
// There is no MFMA anywhere: nothing here is a dense contraction.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>

#include "device_common.hpp"
#include "mlxf_sampler.h"

namespace mlxf {
namespace {

enum { KIND_GREEDY = 0, KIND_TEMP = 1, KIND_KLIST = 2, KIND_KHIST = 3, KIND_TOPP = 4 };
constexpr int LIST = 64;
constexpr int KLIST_MAX = LIST - 1;  // top-k resolved from the best-64 lists
constexpr int CAND_LDS = 4096;
constexpr int CNT_BINS = 4096;  // z-key >> 20: the per-slice top-k threshold bins
constexpr int RBINS = 256;      // radix digit
constexpr unsigned long long MASK40 = (1ull << 40) - 1;
constexpr double HUNIT = 1.0 / 16777216.0;  // 2^-24: histogram mass unit

struct SliceRec {  // four 64-bit words
  float zmax;
  int zarg;
  float mps;  // max z' over the slice
  unsigned int ncand;
  double lse_s;  // sum exp(z - zmax) over the slice
  double msum;   // sum w(z', mps) over the slice
};

struct Args {
  const void* logits;
  long long row_stride;
  int B, V, K_max, S, L;
  const float* T;
  const int* k;
  const float* p;
  const int* tlp;
  const float* u;
  int* out_ids;
  float* out_lp;
  int* out_top_ids;
  float* out_top_lp;
  unsigned int* ctr;
  SliceRec* rec;
  unsigned long long* list;  // [B*S][64] packed (z bits, index)
  unsigned long long* hist;  // [B*S][NBIN]
  uint2* cand;               // [B*S][L]
};

struct Mode {
  int sampling, kk, topp, K, need_lse, want_lp, kind, need_list;
  float Tr, pr, u;
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

__device__ __forceinline__ unsigned long long pack_ent(float v, int i) {
  return pack2(__float_as_uint(v), static_cast<unsigned int>(i));
}

// 64-bit mass added to an LDS counter; one atomic per wave when every active
// lane adds to the same counter (the common case: candidates come in slice
// order, and ties share digits).
__device__ __forceinline__ void lds_add_agg(unsigned long long* base, int idx, unsigned long long q,
                                            bool act) {
  const unsigned long long bal = __ballot(act);
  if (!bal) return;
  const int first = __ffsll(static_cast<long long>(bal)) - 1;
  const int i0 = rdl(idx, first);
  if (__ballot(act && idx != i0) == 0) {
    const unsigned long long s = wave_sum(act ? q : 0ull);
    if ((threadIdx.x & 63) == first && s) atomicAdd(base + i0, s);
  } else if (act && q) {
    atomicAdd(base + idx, q);
  }
}
__device__ __forceinline__ void lds_cnt_agg(unsigned int* base, int idx, bool act) {
  const unsigned long long bal = __ballot(act);
  if (!bal) return;
  const int first = __ffsll(static_cast<long long>(bal)) - 1;
  const int i0 = rdl(idx, first);
  if (__ballot(act && idx != i0) == 0) {
    if ((threadIdx.x & 63) == first) atomicAdd(base + i0, static_cast<unsigned int>(__popcll(bal)));
  } else if (act) {
    atomicAdd(base + idx, 1u);
  }
}

// ------------------------------------------------------------ shared memory --

union Region0 {  // 32 KB
  uint2 cand[CAND_LDS];
  TopEnt surv[CAND_LDS];  // >= 64 * EPT: the most elements that can reach theta
};
union Region1 {  // 16 KB
  unsigned int cnt[CNT_BINS];
  unsigned long long hist[NBIN];
  struct {
    double sp[MAX_S * WAVES];
    unsigned long long sq[MAX_S * WAVES];
  } pass;
};
struct Small {
  Args args;
  Mode md;
  TopEnt lists[WAVES * LIST];  // tree merges
  float rf[WAVES];
  int ri[WAVES];
  double rd[WAVES + 1];
  double rd2[WAVES];
  unsigned long long ru[WAVES + 1];
  int rint[WAVES + 1];
  unsigned int ticket;
  float thv;
  int thi;
  float zmax;
  int zarg;
  double lse;
  float Mp;
  float szmax[MAX_S];
  int szarg[MAX_S];
  double slse[MAX_S];
  unsigned int ncnd[MAX_S];
  float mps[MAX_S];
  double scale[MAX_S];
  double msum[MAX_S];
  int off[MAX_S + 1];
  double side[MAX_S];
  unsigned long long inR[MAX_S];
  unsigned long long keepq[MAX_S];
  double keep[MAX_S];
  TopEnt mlist[LIST];  // the row's merged best-64
  unsigned int rc[RBINS];
  unsigned long long rm[RBINS];
  int sel[16];
  unsigned long long selu[4];
  double seld[4];
  unsigned int ncand;
  unsigned int kmin, kmax;
  int found;
  int pos_hi, pos_lo, pos_last;
};

// A row's candidate list: in LDS, in global memory contiguous, or in global
// memory as the per-slice regions of the first pass (located through off[]).
struct CandView {
  uint2* l;
  uint2* g;
  const int* off;  // nullptr: g is contiguous
  int S, L;
  __device__ __forceinline__ uint2* at(int c) const {
    if (!off) return g + c;
    int lo = 0, hi = S;
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (off[mid] <= c)
        lo = mid;
      else
        hi = mid;
    }
    return g + static_cast<size_t>(lo) * L + (c - off[lo]);
  }
  // candidate c (global entries may come from other workgroups)
  __device__ __forceinline__ uint2 get(int c) const { return l ? l[c] : ld_dev2(at(c)); }
};

// --------------------------------------------------- radix selection (block) --
//
// One selection over the candidates that satisfy `part(e)`, on the field
// F(e) = e.x (key) or e.y (index), scanning values in descending or ascending
// order, measuring either counts or fixed-point masses wq(e).  It returns the
// first value v in scan order at which  before + measure(v) >= target
// (> target when strict) with measure(v) > 0, where `before` is the measure of
// the values that precede v; *before_out gets `before`, *gcount the number of
// participants equal to v.  In mass mode, when no value qualifies (the target
// exceeds the total), the last value in scan order is returned and *none is
// set.  Rounds of 8-bit digits; the leading digits the participants all share
// are skipped.  Must be called by the whole workgroup.
template <bool BY_KEY, bool DESC, bool MASS, typename PART, typename WQ>
__device__ unsigned int radix_select(const CandView& cv, int n, PART part, WQ wq,
                                     unsigned long long target, bool strict, Small& sh,
                                     unsigned long long* before_out, unsigned int* gcount,
                                     bool* none) {
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  // ---- range of the field over participants, and their count and measure
  unsigned int lo = 0xffffffffu, hi = 0u;
  unsigned long long cnt_all = 0, mass_all = 0;
  for (int c = tid; c < n; c += THREADS) {
    const uint2 e = cv.get(c);
    if (part(e)) {
      const unsigned int f = BY_KEY ? e.x : e.y;
      lo = min(lo, f);
      hi = max(hi, f);
      cnt_all += 1;
      if (MASS) mass_all += wq(e);
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
  cnt_all = block_sum<unsigned long long>(cnt_all, sh.ru);
  if (MASS) mass_all = block_sum<unsigned long long>(mass_all, sh.ru);
  lo = sh.kmin;
  hi = sh.kmax;
  __syncthreads();
  if (cnt_all == 0) {
    *before_out = 0;
    *gcount = 0;
    *none = true;
    return 0;
  }
  const unsigned long long tot = MASS ? mass_all : cnt_all;
  const bool reach = strict ? tot > target : tot >= target;
  if (lo == hi) {  // a single value
    *before_out = 0;
    *gcount = static_cast<unsigned int>(cnt_all);
    *none = MASS && !reach;
    return lo;
  }
  if (MASS && !reach) {
    // nothing qualifies: the last value in scan order, everything before it
    const unsigned int v = DESC ? lo : hi;
    unsigned long long cv_cnt = 0, cv_mass = 0;
    for (int c = tid; c < n; c += THREADS) {
      const uint2 e = cv.get(c);
      if (part(e) && (BY_KEY ? e.x : e.y) == v) {
        cv_cnt += 1;
        cv_mass += wq(e);
      }
    }
    cv_cnt = block_sum<unsigned long long>(cv_cnt, sh.ru);
    cv_mass = block_sum<unsigned long long>(cv_mass, sh.ru);
    *before_out = mass_all - cv_mass;
    *gcount = static_cast<unsigned int>(cv_cnt);
    *none = true;
    return v;
  }
  const unsigned int diff = lo ^ hi;
  const int top = 31 - __clz(static_cast<int>(diff));
  int shift = (top >> 3) << 3;
  unsigned int mask = shift + 8 >= 32 ? 0u : ~((1u << (shift + 8)) - 1u);
  unsigned int prefix = lo & mask;
  unsigned long long before = 0;
  unsigned int g = 0;
  for (; shift >= 0; shift -= 8) {
    for (int d = tid; d < RBINS; d += THREADS) {
      sh.rc[d] = 0u;
      if (MASS) sh.rm[d] = 0ull;
    }
    __syncthreads();
    for (int base = 0; base < n; base += THREADS) {
      const int c = base + tid;
      uint2 e = make_uint2(0u, 0u);
      bool act = false;
      if (c < n) {
        e = cv.get(c);
        const unsigned int f = BY_KEY ? e.x : e.y;
        act = part(e) && (f & mask) == prefix;
      }
      const unsigned int f = BY_KEY ? e.x : e.y;
      const int d = static_cast<int>((f >> shift) & 255u);
      lds_cnt_agg(sh.rc, d, act);
      if (MASS) lds_add_agg(sh.rm, d, act ? wq(e) : 0ull, act);
    }
    __syncthreads();
    if (wid == 0) {
      // lane l owns scan positions 4l..4l+3
      unsigned long long val[4];
      unsigned int cnt[4];
      unsigned long long sum = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int pos = 4 * lane + q;
        const int d = DESC ? RBINS - 1 - pos : pos;
        cnt[q] = sh.rc[d];
        val[q] = MASS ? sh.rm[d] : static_cast<unsigned long long>(cnt[q]);
        sum += val[q];
      }
      const unsigned long long inc = wave_incl_scan(sum);
      unsigned long long run = inc - sum;
      const unsigned long long tg = target > before ? target - before : 0ull;
      int found = 4 * 64, lastne = -1;
      unsigned long long bef = 0, bef_last = 0;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int pos = 4 * lane + q;
        if (found == 4 * 64 && val[q] > 0 && (strict ? run + val[q] > tg : run + val[q] >= tg)) {
          found = pos;
          bef = run;
        }
        if (cnt[q] > 0) {
          lastne = pos;
          bef_last = run;
        }
        run += val[q];
      }
      int best = wave_min(found);
      const int lbest = wave_max(lastne);
      // the total reaches the target, so some digit qualifies; the last
      // non-empty digit only guards against a total that rounding made short
      unsigned long long b;
      if (best < 4 * 64) {
        b = rdl(bef, best >> 2);
      } else {
        best = lbest < 0 ? 0 : lbest;
        b = rdl(bef_last, best >> 2);
      }
      if (lane == 0) {
        const int d = DESC ? RBINS - 1 - best : best;
        sh.sel[0] = d;
        sh.sel[2] = static_cast<int>(sh.rc[d]);
        sh.selu[0] = b;
      }
    }
    __syncthreads();
    prefix |= static_cast<unsigned int>(sh.sel[0]) << shift;
    mask |= 255u << shift;
    before += sh.selu[0];
    g = static_cast<unsigned int>(sh.sel[2]);
    __syncthreads();
  }
  *before_out = before;
  *gcount = g;
  *none = false;
  return prefix;
}

// -------------------------------------------------- candidate-set finishing --

// Top-k (then optionally top-p) and the draw, all on a candidate set that holds
// every element whose z' reaches the row's k-th largest z' (keys are z' keys).
// Returns the drawn index.
__device__ int resolve_topk(const Mode& md, const CandView& cv, int n, float Mp, Small& sh) {
  auto wq = [Mp](uint2 e) { return quant(wexp(key2f(e.x), Mp)); };
  auto all = [](uint2) { return true; };
  unsigned long long bef;
  unsigned int g;
  bool none;
  // (1) k-th largest key, with multiplicity
  const unsigned int tau = radix_select<true, true, false>(
      cv, n, all, wq, static_cast<unsigned long long>(md.kk), false, sh, &bef, &g, &none);
  // (2) mass of the top-k set
  unsigned long long wk = 0;
  for (int c = threadIdx.x; c < n; c += THREADS) {
    const uint2 e = cv.get(c);
    if (e.x >= tau) wk += wq(e);
  }
  wk = block_sum<unsigned long long>(wk, sh.ru);
  unsigned int vkey = tau;
  int idx_cut = INT_MAX;
  unsigned long long Wf = wk;
  if (md.topp) {
    // (3) nucleus cutoff: keep while the mass before an element is < p * W_k
    const unsigned long long PW =
        static_cast<unsigned long long>(ceil(static_cast<double>(md.pr) * static_cast<double>(wk)));
    auto ge_tau = [tau](uint2 e) { return e.x >= tau; };
    unsigned long long pgt;
    vkey = radix_select<true, true, true>(cv, n, ge_tau, wq, PW, false, sh, &pgt, &g, &none);
    const unsigned long long wstar = wq(make_uint2(vkey, 0u));
    unsigned long long t = g;
    if (!none && wstar > 0) {
      const unsigned long long need = PW > pgt ? (PW - pgt + wstar - 1) / wstar : 0ull;
      t = need < t ? need : t;
    }
    if (t == 0) t = 1;
    if (t < g) {  // (4) the t-th smallest index among the ties at the cutoff
      auto eq_v = [vkey](uint2 e) { return e.x == vkey; };
      idx_cut = static_cast<int>(
          radix_select<false, false, false>(cv, n, eq_v, wq, t, false, sh, &bef, &g, &none));
    }
    Wf = pgt + t * wstar;
  }
  // (5) inverse-CDF draw in vocabulary order over the kept set
  unsigned long long T = static_cast<unsigned long long>(static_cast<double>(md.u) * static_cast<double>(Wf));
  if (Wf == 0)
    T = 0;
  else if (T >= Wf)
    T = Wf - 1;
  auto kept = [vkey, idx_cut](uint2 e) {
    return e.x > vkey || (e.x == vkey && static_cast<int>(e.y) <= idx_cut);
  };
  if (Wf == 0) {  // every kept weight underflowed: the lowest kept index
    return static_cast<int>(radix_select<false, false, false>(cv, n, kept, wq, 1ull, false, sh, &bef,
                                                              &g, &none));
  }
  return static_cast<int>(radix_select<false, false, true>(cv, n, kept, wq, T, true, sh, &bef, &g, &none));
}

// ------------------------------------------------------- last-block stages --

// Walk slice s in vocabulary order; the first kept element at which the
// running mass w(z', mps_s) exceeds rem is the draw.  Kept: key(z') > vkey, or
// equal with index <= idx_cut.  Thread t owns EPT consecutive elements, read 8
// at a time (the thread that holds the crossing reads its elements again; they
// are in L2 by then).
template <int DT, int EPT, bool VECOK>
__device__ int final_scan(const Args& a, const Mode& md, const void* row, int s, double rem,
                          unsigned int vkey, int idx_cut, Small& sh) {
  const int tid = threadIdx.x;
  const int b0 = s * a.L;
  const int e0 = min(a.V, b0 + a.L);
  const float mps = sh.mps[s];
  const int my0 = b0 + tid * EPT;
  auto weight = [&](float z, int i) {
    const float zp = fz<DT>(z, md.Tr);
    const unsigned int key = f2key(zp);
    const bool kept = i < e0 && (key > vkey || (key == vkey && i <= idx_cut));
    return kept ? wexp(zp, mps) : 0.0f;
  };
  double sum = 0.0;
  int last_pos = -1;
#pragma unroll 2
  for (int it = 0; it < EPT / VEC; ++it) {
    float z[VEC];
    load8<DT, VECOK>(row, my0 + it * VEC, e0, z);
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const float ww = weight(z[j], my0 + it * VEC + j);
      sum += static_cast<double>(ww);
      if (ww > 0.0f) last_pos = my0 + it * VEC + j;
    }
  }
  double ex, in, tot;
  block_scan<double>(sum, sh.rd, &ex, &in, &tot);
  if (tid == 0) sh.found = -1;
  __syncthreads();
  if (ex <= rem && rem < in) {
    double c = ex;
    int pick = -1;
    for (int it = 0; it < EPT / VEC && pick < 0; ++it) {
      float z[VEC];
      load8<DT, VECOK>(row, my0 + it * VEC, e0, z);
#pragma unroll
      for (int j = 0; j < VEC; ++j) {
        const float ww = weight(z[j], my0 + it * VEC + j);
        c += static_cast<double>(ww);
        if (pick < 0 && c > rem && ww > 0.0f) pick = my0 + it * VEC + j;
      }
    }
    sh.found = pick < 0 ? last_pos : pick;  // rounding inside the thread: its last positive element
  }
  __syncthreads();
  int id = sh.found;
  if (id < 0) {  // rem at or past the slice total (fp64 rounding): last kept element
    const int lp = wave_max(last_pos);
    if ((tid & 63) == 0) sh.rint[tid >> 6] = lp;
    __syncthreads();
    if (tid == 0) {
      int m = -1;
      for (int w2 = 0; w2 < WAVES; ++w2) m = max(m, sh.rint[w2]);
      sh.found = m < 0 ? b0 : m;
    }
    __syncthreads();
    id = sh.found;
  }
  return id;
}

template <int DT>
__device__ void write_sampled(const Args& a, const Mode& md, const void* row, int r, int id,
                              const Small& sh) {
  if (threadIdx.x != 0) return;
  a.out_ids[r] = id;
  if (a.out_lp)
    a.out_lp[r] = md.want_lp ? static_cast<float>(static_cast<double>(ld1<DT>(row, id)) - sh.lse)
                             : NAN;
}

// Index of the slice holding u * (total kept mass) and the remaining target in
// that slice's own units.  keep[t] are slice-unit masses, scale[t] converts them
// to row units.
__device__ void pick_slice(const double* keep, const double* scale, int S, float u, int* sst_out,
                           double* rem_out) {
  double W = 0.0;
  for (int t = 0; t < S; ++t) W += keep[t] * scale[t];
  const double T = static_cast<double>(u) * W;
  double cum = 0.0, before = 0.0;
  int sst = -1;
  for (int t = 0; t < S; ++t) {
    const double m = keep[t] * scale[t];
    if (m > 0.0) {
      sst = t;
      before = cum;
      if (cum + m > T) break;
    }
    cum += m;
  }
  if (sst < 0) {
    sst = 0;
    before = 0.0;
  }
  *sst_out = sst;
  *rem_out = scale[sst] > 0.0 ? (T - before) / scale[sst] : 0.0;
}

// Temperature only: all elements kept.
template <int DT, int EPT, bool VECOK>
__device__ void finish_temp(const Args& a, const Mode& md, const void* row, int r, Small& sh) {
  if (threadIdx.x == 0) {
    int sst;
    double rem;
    pick_slice(sh.msum, sh.scale, a.S, md.u, &sst, &rem);
    sh.sel[0] = sst;
    sh.seld[0] = rem;
  }
  __syncthreads();
  const int id = final_scan<DT, EPT, VECOK>(a, md, row, sh.sel[0], sh.seld[0], 0u, INT_MAX, sh);
  write_sampled<DT>(a, md, row, r, id, sh);
}

// Top-k <= 63 from the row's merged best-64 list, by one wave.  Returns false
// when the list may miss elements tied at the k-th value of z' (then the caller
// extracts the candidates from the row).
template <int DT>
__device__ bool klist_resolve(const Mode& md, float Mp, const Small& sh, int* id_out) {
  const int lane = threadIdx.x & 63;
  const float lv = sh.mlist[lane].v;
  const int li = sh.mlist[lane].i;
  const bool real = li != INT_MAX;
  const float zp = real ? fz<DT>(lv, md.Tr) : -INFINITY;
  const float tau = rdl(zp, md.kk - 1);
  const int last_i = rdl(li, LIST - 1);
  const float last_zp = rdl(zp, LIST - 1);
  // every element with z' >= tau is in the list unless the list's last entry reaches tau
  if (last_i != INT_MAX && !(last_zp < tau)) return false;
  const bool in_k = real && zp >= tau;
  float sv = in_k ? zp : -INFINITY;
  int si = in_k ? li : INT_MAX;
  wave_sort(sv, si);  // (z' desc, index asc)
  const bool k1 = si != INT_MAX;
  const unsigned long long w = k1 ? quant(wexp(sv, Mp)) : 0ull;
  const unsigned long long incl = wave_incl_scan(w);
  const unsigned long long Wk = rdl(incl, 63);
  bool keep = k1;
  if (md.topp) {
    const unsigned long long PW =
        static_cast<unsigned long long>(ceil(static_cast<double>(md.pr) * static_cast<double>(Wk)));
    keep = k1 && (incl - w) < PW;
  }
  const unsigned long long wf = keep ? w : 0ull;
  const unsigned long long Wf = wave_sum(wf);
  unsigned long long T = static_cast<unsigned long long>(static_cast<double>(md.u) * static_cast<double>(Wf));
  if (Wf == 0)
    T = 0;
  else if (T >= Wf)
    T = Wf - 1;
  // mass of kept entries with index <= mine, in vocabulary order
  unsigned long long cum = 0;
  for (int q = 0; q < 64; ++q) {
    const unsigned int wlo = __builtin_amdgcn_readlane(static_cast<unsigned int>(wf), q);
    const unsigned int whi = __builtin_amdgcn_readlane(static_cast<unsigned int>(wf >> 32), q);
    const int iq = __builtin_amdgcn_readlane(si, q);
    if (iq <= si) cum += pack2(wlo, whi);
  }
  const int cand = wave_min((keep && (Wf == 0 || (wf > 0 && cum > T))) ? si : INT_MAX);
  *id_out = cand == INT_MAX ? rdl(si, 0) : cand;
  return true;
}

// Compare-only pass over the row (the finishing workgroup alone): elements with
// z key in [klo, khi) become candidates (z' key, index), and the in-range mass
// of slice t (2^-42 units of w(z', mps_t)) goes to r1.pass.sq[t * WAVES + wave];
// when `sum_side` is 1 (above: z key >= khi) or 2 (below: z key < klo) the mass
// of that side goes to r1.pass.sp.  has_hi false: no upper bound.  G slices'
// loads are in flight at once.
template <int DT, int EPT, bool VECOK>
__device__ void row_pass(const Args& a, const Mode& md, const void* row, int r, unsigned int klo,
                         bool has_hi, unsigned int khi, int sum_side, Region0& r0, Region1& r1,
                         Small& sh) {
  constexpr int NIT = EPT / VEC;
  // slices whose raw loads are in flight together: about 64 VGPRs of raw data
  constexpr int G0 = (DT == MLXF_DTYPE_F32 ? 64 : 128) / EPT;
  constexpr int G = G0 > 8 ? 8 : G0;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int S = a.S;
  uint2* g = a.cand + static_cast<size_t>(r) * S * a.L;
#pragma unroll 1
  for (int t0 = 0; t0 < S; t0 += G) {
    Raw8<DT> q[G][NIT];
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const int t = t0 + gi;
      if (t < S) {
        const int b0 = t * a.L, e0 = min(a.V, b0 + a.L);
#pragma unroll
        for (int it = 0; it < NIT; ++it) load_raw<DT, VECOK>(row, b0 + it * CHUNK + tid * VEC, e0, q[gi][it]);
      }
    }
#pragma unroll
    for (int gi = 0; gi < G; ++gi) {
      const int t = t0 + gi;
      if (t < S) {
        const int b0 = t * a.L, e0 = min(a.V, b0 + a.L);
        const float mps = sh.mps[t];
        float part = 0.0f;
        unsigned long long pq = 0;
#pragma unroll
        for (int it = 0; it < NIT; ++it) {
          float z[VEC];
          decode8<DT>(q[gi][it], z);
          const int i0 = b0 + it * CHUNK + tid * VEC;
#pragma unroll
          for (int j = 0; j < VEC; ++j) {
            const int i = i0 + j;
            const bool valid = i < e0;
            const unsigned int zk = f2key(z[j]);
            const bool above = valid && has_hi && zk >= khi;
            const bool inr = valid && !above && zk >= klo;
            const bool side = sum_side == 1 ? above : (sum_side == 2 && valid && !above && !inr);
            unsigned int zpk = 0;
            if (side || inr) {  // most elements need neither the division nor the exp
              const float zp = fz<DT>(z[j], md.Tr);
              const float w = wexp(zp, mps);
              if (side) part += w;
              if (inr) pq += quant(w);
              zpk = f2key(zp);
            }
            const unsigned long long bal = __ballot(inr);
            if (bal) {
              unsigned int basepos = 0;
              if (lane == 0) basepos = atomicAdd(&sh.ncand, static_cast<unsigned int>(__popcll(bal)));
              basepos = rdl(basepos, 0);
              if (inr) {
                const unsigned int pos =
                    basepos + __builtin_amdgcn_mbcnt_hi(static_cast<unsigned int>(bal >> 32),
                                                        __builtin_amdgcn_mbcnt_lo(static_cast<unsigned int>(bal), 0u));
                const uint2 ent = make_uint2(zpk, static_cast<unsigned int>(i));
                st_dev(g + pos, ent);
                if (pos < CAND_LDS) r0.cand[pos] = ent;
              }
            }
          }
        }
        const double pd = wave_sum(static_cast<double>(part));
        pq = wave_sum(pq);
        if (lane == 0) {
          r1.pass.sp[t * WAVES + wid] = pd;
          r1.pass.sq[t * WAVES + wid] = pq;
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // candidate stores complete before other waves read them
  __syncthreads();
}

// Top-k from candidates of the first pass (k > 63), or -- when the best-64 list
// cannot decide a k <= 63 row -- from candidates extracted from the row now.
template <int DT, int EPT, bool VECOK>
__device__ void finish_topk(const Args& a, const Mode& md, const void* row, int r, bool from_row,
                            Region0& r0, Region1& r1, Small& sh) {
  const int tid = threadIdx.x;
  const int S = a.S;
  CandView cv;
  int n;
  if (from_row) {
    // every element with z' >= z'(list entry k-1) -- i.e. z key >= g(that z')
    if (tid == 0) {
      const float tau_z = sh.mlist[md.kk - 1].v;
      sh.sel[4] = static_cast<int>(gkey<DT>(fz<DT>(tau_z, md.Tr), md.Tr));
      sh.ncand = 0;
    }
    __syncthreads();
    row_pass<DT, EPT, VECOK>(a, md, row, r, static_cast<unsigned int>(sh.sel[4]), false, 0u, 0, r0,
                             r1, sh);
    n = static_cast<int>(sh.ncand);
    cv.l = n <= CAND_LDS ? r0.cand : nullptr;
    cv.g = a.cand + static_cast<size_t>(r) * S * a.L;
    cv.off = nullptr;
  } else {
    if (tid == 0) {
      int o = 0;
      for (int t = 0; t < S; ++t) {
        sh.off[t] = o;
        o += static_cast<int>(sh.ncnd[t]);
      }
      sh.off[S] = o;
    }
    __syncthreads();
    n = sh.off[S];
    uint2* g = a.cand + static_cast<size_t>(r) * S * a.L;
    const bool in_lds = n <= CAND_LDS;
    for (int t = 0; t < S; ++t) {  // z key -> z' key
      const int o = sh.off[t], cnt = sh.off[t + 1] - o;
      uint2* src = g + static_cast<size_t>(t) * a.L;
      for (int j = tid; j < cnt; j += THREADS) {
        uint2 e = ld_dev2(src + j);
        e.x = f2key(fz<DT>(key2f(e.x), md.Tr));
        if (in_lds)
          r0.cand[o + j] = e;
        else
          st_dev(src + j, e);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);  // global rewrites complete before other waves read them
    __syncthreads();
    cv.l = in_lds ? r0.cand : nullptr;
    cv.g = g;
    cv.off = sh.off;
  }
  cv.S = S;
  cv.L = a.L;
  const int id = resolve_topk(md, cv, n, sh.Mp, sh);
  write_sampled<DT>(a, md, row, r, id, sh);
}

// Top-p without top-k, in phases that hand their results on through LDS so
// that little stays live in registers across phases:
//   A: combined histogram (row units) with the bound of its truncation error;
//      the bracket R = [blo, bhi] of bins that must hold the nucleus boundary;
//      the side of R with fewer elements.
//   B: R's edges as z-key thresholds (no division in the comparisons).
//   C: compare-only pass over the row.
//   D: mass above R per slice; check that R brackets the boundary (else redo
//      with R = the whole row).
//   E: exact cutoff and tie cut among R's elements, kept mass per slice, the
//      slice that holds the draw, and the walk of that slice.
template <int DT, int EPT, bool VECOK>
__device__ void finish_topp(const Args& a, const Mode& md, const void* row, int r, Region0& r0,
                            Region1& r1, Small& sh) {
  const int tid = threadIdx.x;
  const int S = a.S;

  // ---- A: thread t owns descending positions PB*t .. PB*t+PB-1 (bins NBIN-1-PB*t ...)
  constexpr int PB = NBIN / THREADS;
  {
    const size_t hb = static_cast<size_t>(r) * S * NBIN;
    unsigned int c[PB];
    double m[PB], e[PB];
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      c[q] = 0u;
      m[q] = 0.0;
      e[q] = 0.0;
      const int b = NBIN - 1 - (PB * tid + q);
#pragma unroll 8
      for (int t = 0; t < S; ++t) {
        const unsigned long long h = ld_dev(a.hist + hb + static_cast<size_t>(t) * NBIN + b);
        const unsigned int ct = static_cast<unsigned int>(h >> 40);
        c[q] += ct;
        m[q] += static_cast<double>(h & MASK40) * HUNIT * sh.scale[t];
        e[q] += static_cast<double>(ct) * HUNIT * sh.scale[t];
      }
    }
    if (tid == 0) {
      double W = 0.0;
      for (int t = 0; t < S; ++t) W += sh.msum[t] * sh.scale[t];
      sh.seld[2] = static_cast<double>(md.pr) * W;  // p * W, row units
      sh.pos_hi = NBIN;
      sh.pos_lo = NBIN;
      sh.pos_last = -1;
    }
    double sA = 0.0, sU = 0.0;
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      sA += m[q];
      sU += m[q] + e[q];
    }
    double exA, inA, totA, exU, inU, totU;
    block_scan<double>(sA, sh.rd, &exA, &inA, &totA);
    block_scan<double>(sU, sh.rd, &exU, &inU, &totU);
    const double PW = sh.seld[2];
    // first position whose cumulative upper bound reaches p*W: the boundary is
    // not above it; first position whose cumulative lower bound reaches it:
    // the boundary is not below it
    const double t_hi = PW * (1.0 - 1e-9), t_lo = PW * (1.0 + 1e-9);
    int ph = NBIN, pl = NBIN, last = -1;
    double runA = exA, runU = exU;
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      runA += m[q];
      runU += m[q] + e[q];
      if (c[q] > 0) {
        if (ph == NBIN && runU >= t_hi) ph = PB * tid + q;
        if (pl == NBIN && runA >= t_lo) pl = PB * tid + q;
        last = PB * tid + q;
      }
    }
    if (ph < NBIN) atomicMin(&sh.pos_hi, ph);
    if (pl < NBIN) atomicMin(&sh.pos_lo, pl);
    if (last >= 0) atomicMax(&sh.pos_last, last);
    __syncthreads();
    int p_hi = sh.pos_hi, p_lo = sh.pos_lo;
    const int p_last = sh.pos_last < 0 ? NBIN - 1 : sh.pos_last;
    if (p_hi > p_last) p_hi = p_last;
    if (p_lo > p_last) p_lo = p_last;
    // positions count down from the top bin: bhi = NBIN-1-p_hi >= blo = NBIN-1-p_lo
    int ca = 0, cb = 0;
#pragma unroll
    for (int q = 0; q < PB; ++q) {
      const int pos = PB * tid + q;
      if (pos < p_hi) ca += static_cast<int>(c[q]);
      if (pos > p_lo) cb += static_cast<int>(c[q]);
    }
    ca = block_sum<int>(ca, sh.rint);
    cb = block_sum<int>(cb, sh.rint);
    if (tid == 0) {
      sh.sel[2] = NBIN - 1 - p_lo;  // blo
      sh.sel[3] = NBIN - 1 - p_hi;  // bhi
      sh.sel[7] = ca <= cb ? 1 : 2;  // sum the side with fewer elements
    }
    __syncthreads();
  }

  for (int attempt = 0; attempt < 2; ++attempt) {
    // ---- B
    if (tid == 0) {
      const int blo = sh.sel[2], bhi = sh.sel[3];
      const unsigned int klo_edge = max(static_cast<unsigned int>(blo) << 21, KEY_NEG_INF);
      sh.sel[4] = static_cast<int>(attempt == 0 ? gkey<DT>(key2f(klo_edge), md.Tr) : 0u);
      const unsigned int hi_edge = static_cast<unsigned int>(bhi + 1) << 21;
      const bool has_hi = attempt == 0 && bhi < NBIN - 1 && hi_edge <= KEY_POS_INF;
      sh.sel[5] = has_hi ? 1 : 0;
      sh.sel[6] = static_cast<int>(has_hi ? gkey<DT>(key2f(hi_edge), md.Tr) : 0u);
      sh.sel[8] = attempt == 0 ? sh.sel[7] : 0;  // R = whole row: no side to sum
      sh.ncand = 0;
    }
    __syncthreads();
    // ---- C
    row_pass<DT, EPT, VECOK>(a, md, row, r, static_cast<unsigned int>(sh.sel[4]), sh.sel[5] != 0,
                             static_cast<unsigned int>(sh.sel[6]), sh.sel[8], r0, r1, sh);
    // ---- D
    if (tid < S) {
      double sd = 0.0;
      unsigned long long sq = 0;
      for (int w2 = 0; w2 < WAVES; ++w2) {
        sd += r1.pass.sp[tid * WAVES + w2];
        sq += r1.pass.sq[tid * WAVES + w2];
      }
      sh.side[tid] = sd;
      sh.inR[tid] = sq;
      sh.keepq[tid] = 0ull;
    }
    __syncthreads();
    const int n = static_cast<int>(sh.ncand);
    CandView cv;
    cv.l = n <= CAND_LDS ? r0.cand : nullptr;
    cv.g = a.cand + static_cast<size_t>(r) * S * a.L;
    cv.off = nullptr;
    cv.S = S;
    cv.L = a.L;
    const float Mp = sh.Mp;
    auto wq = [Mp](uint2 e) { return quant(wexp(key2f(e.x), Mp)); };
    if (tid == 0) {
      const int side = sh.sel[8];
      double pa = 0.0, inr_tot = 0.0;
      for (int t = 0; t < S; ++t) {
        const double inr = static_cast<double>(sh.inR[t]) * QUNIT;
        const double ab = side == 1 ? sh.side[t] : (side == 2 ? sh.msum[t] - sh.side[t] - inr : 0.0);
        sh.keep[t] = ab < 0.0 ? 0.0 : ab;  // above-R mass, slice units
        pa += sh.keep[t] * sh.scale[t];
        inr_tot += inr * sh.scale[t];
      }
      const double need = sh.seld[2] - pa;  // nucleus mass still to cover inside R, row units
      const bool bracketed = need > 0.0 && need <= inr_tot * (1.0 + 1e-9) + 1e-12;
      sh.sel[9] = bracketed ? 1 : 0;
      const double nq = need / QUNIT;
      sh.selu[1] = nq <= 1.0 ? 1ull : static_cast<unsigned long long>(ceil(nq));
    }
    __syncthreads();
    if (sh.sel[9] == 0 && attempt == 0) {  // R missed the boundary: R = whole row
      if (tid == 0) {
        sh.sel[2] = 0;
        sh.sel[3] = NBIN - 1;
      }
      __syncthreads();
      continue;
    }
    // ---- E
    const unsigned long long target = sh.selu[1];
    unsigned long long pgt, bef;
    unsigned int g_cnt;
    bool all_kept;
    auto any = [](uint2) { return true; };
    const unsigned int vkey =
        radix_select<true, true, true>(cv, n, any, wq, target, false, sh, &pgt, &g_cnt, &all_kept);
    const unsigned long long wstar = wq(make_uint2(vkey, 0u));
    unsigned long long tk = g_cnt;
    if (!all_kept && wstar > 0) {
      const unsigned long long nd = target > pgt ? (target - pgt + wstar - 1) / wstar : 0ull;
      tk = nd < tk ? nd : tk;
    }
    if (tk == 0) tk = 1;
    int idx_cut = INT_MAX;
    if (tk < g_cnt) {
      auto eq_v = [vkey](uint2 e) { return e.x == vkey; };
      unsigned int g2;
      bool none2;
      idx_cut = static_cast<int>(
          radix_select<false, false, false>(cv, n, eq_v, wq, tk, false, sh, &bef, &g2, &none2));
    }
    for (int base = 0; base < n; base += THREADS) {
      const int c = base + tid;
      bool kept = false;
      int st = 0;
      unsigned long long q = 0;
      if (c < n) {
        const uint2 e = cv.get(c);
        kept = e.x > vkey || (e.x == vkey && static_cast<int>(e.y) <= idx_cut);
        st = static_cast<int>(e.y) / a.L;
        q = kept ? quant(wexp(key2f(e.x), sh.mps[st])) : 0ull;
      }
      lds_add_agg(sh.keepq, st, q, kept);
    }
    __syncthreads();
    if (tid == 0) {
      for (int t = 0; t < S; ++t) sh.keep[t] += static_cast<double>(sh.keepq[t]) * QUNIT;
      int sst;
      double rem;
      pick_slice(sh.keep, sh.scale, S, md.u, &sst, &rem);
      sh.sel[0] = sst;
      sh.seld[1] = rem;
    }
    __syncthreads();
    const int id = final_scan<DT, EPT, VECOK>(a, md, row, sh.sel[0], sh.seld[1], vkey, idx_cut, sh);
    write_sampled<DT>(a, md, row, r, id, sh);
    return;
  }
}

// Everything the last slice of a row does.
template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ void finish_row(int r, Region0& r0, Region1& r1, Small& sh) {
  const Args& a = sh.args;
  const Mode& md = sh.md;  // in LDS: callees that are not inlined take it by reference
  const void* row = row_ptr<DT>(a, r);
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int S = a.S;

  if (tid < S) {
    const unsigned long long* rp = reinterpret_cast<const unsigned long long*>(a.rec + (r * S + tid));
    const unsigned long long w0 = ld_dev(rp + 0), w1 = ld_dev(rp + 1);
    sh.szmax[tid] = __uint_as_float(static_cast<unsigned int>(w0));
    sh.szarg[tid] = static_cast<int>(w0 >> 32);
    sh.mps[tid] = __uint_as_float(static_cast<unsigned int>(w1));
    sh.ncnd[tid] = static_cast<unsigned int>(w1 >> 32);
    sh.slse[tid] = __longlong_as_double(static_cast<long long>(ld_dev(rp + 2)));
    sh.msum[tid] = __longlong_as_double(static_cast<long long>(ld_dev(rp + 3)));
  }
  // the row's best 64: wave w merges the lists of slices w, w + 16, ...; then a tree
  if (md.need_list) {
    float lv = -INFINITY;
    int li = INT_MAX;
    for (int t = wid; t < S; t += WAVES) {
      const unsigned long long w = ld_dev(a.list + (static_cast<size_t>(r) * S + t) * LIST + lane);
      wave_list_merge(lv, li, __uint_as_float(static_cast<unsigned int>(w)), static_cast<int>(w >> 32));
    }
    tree_merge(lv, li, sh.lists, S < WAVES ? S : WAVES);
    if (wid == 0) {
      sh.mlist[lane].v = lv;
      sh.mlist[lane].i = li;
    }
  }
  __syncthreads();
  if (wid == 0) {
    const float zm = lane < S ? sh.szmax[lane] : -INFINITY;
    const int za = lane < S ? sh.szarg[lane] : INT_MAX;
    float rm = zm;
    int ra = za;
    wave_best(rm, ra);
    double part = (lane < S && md.need_lse) ? sh.slse[lane] * wexp_d(zm, rm) : 0.0;
    part = wave_sum(part);
    const float Mp = md.sampling ? fz<DT>(rm, md.Tr) : 0.0f;
    if (lane < S && md.sampling) sh.scale[lane] = wexp_d(sh.mps[lane], Mp);
    if (lane == 0) {
      sh.zmax = rm;
      sh.zarg = ra;
      sh.lse = md.need_lse ? static_cast<double>(rm) + log(part) : static_cast<double>(NAN);
      sh.Mp = Mp;
    }
  }
  __syncthreads();

  if (tid == 0 && md.kind == KIND_GREEDY) {
    a.out_ids[r] = sh.zarg;
    if (a.out_lp)
      a.out_lp[r] = md.want_lp ? static_cast<float>(static_cast<double>(sh.zmax) - sh.lse) : NAN;
  }
  if (a.K_max > 0 && tid < a.K_max) {  // top_logprobs: the first K of the best-64
    const size_t o = static_cast<size_t>(r) * a.K_max + tid;
    if (tid < md.K) {
      a.out_top_ids[o] = sh.mlist[tid].i;
      a.out_top_lp[o] = static_cast<float>(static_cast<double>(sh.mlist[tid].v) - sh.lse);
    } else {
      a.out_top_ids[o] = -1;
      a.out_top_lp[o] = -INFINITY;
    }
  }

  if (md.topp && !(md.pr > 0.0f)) {
    // p rounds to 0 in the logits dtype: the nucleus keeps nothing, every
    // logit is masked, and the draw is uniform over the vocabulary
    if (tid == 0) {
      const double x = floor(static_cast<double>(md.u) * static_cast<double>(a.V));
      write_sampled<DT>(a, md, row, r, x < a.V - 1 ? static_cast<int>(x) : a.V - 1, sh);
    }
  } else if (md.kind == KIND_TEMP) {
    finish_temp<DT, EPT, VECOK>(a, md, row, r, sh);
  } else if (md.kind == KIND_KLIST) {
    if (wid == 0) {
      int id = -1;
      const bool ok = klist_resolve<DT>(md, sh.Mp, sh, &id);
      if (lane == 0) {
        sh.sel[10] = ok ? 1 : 0;
        sh.sel[11] = id;
      }
    }
    __syncthreads();
    if (sh.sel[10])
      write_sampled<DT>(a, md, row, r, sh.sel[11], sh);
    else
      finish_topk<DT, EPT, VECOK>(a, md, row, r, true, r0, r1, sh);
  } else if (md.kind == KIND_KHIST) {
    finish_topk<DT, EPT, VECOK>(a, md, row, r, false, r0, r1, sh);
  } else if (md.kind == KIND_TOPP) {
    finish_topp<DT, EPT, VECOK>(a, md, row, r, r0, r1, sh);
  }
}

// =================================================================== kernel ==

template <int DT, int EPT, bool VECOK>
__global__ __launch_bounds__(THREADS, 2) void k_sample(Args a) {
  __shared__ Region0 r0;
  __shared__ Region1 r1;
  __shared__ Small sh;

  const int s = blockIdx.x, r = blockIdx.y;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int S = a.S;
  const Mode md = decode<DT>(a, r);
  const void* row = row_ptr<DT>(a, r);
  const int beg = s * a.L;
  const int end = min(a.V, beg + a.L);
  constexpr int NIT = EPT / VEC;

  float v[EPT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) load8<DT, VECOK>(row, beg + it * CHUNK + tid * VEC, end, &v[it * VEC]);
#define MLXF_IDX(e) (beg + ((e) / VEC) * CHUNK + tid * VEC + ((e) % VEC))

  // Histograms are cleared while the loads are in flight.  The pass has two
  // barriers: B1 publishes the wave maxima (and list thresholds), B2 the
  // argmax, the sums and the survivors.
  if (md.kind == KIND_TOPP) {
    for (int b = tid; b < NBIN; b += THREADS) r1.hist[b] = 0ull;
  } else if (md.kind == KIND_KHIST) {
    for (int b = tid; b < CNT_BINS; b += THREADS) r1.cnt[b] = 0u;
  }
  if (tid == 0) sh.ncand = 0u;

  // ---- thread max; each wave's max and, for the best-64 list, the wave's 16th
  // largest thread maximum (a bisection on the key with ballots)
  float tmax = v[0];
#pragma unroll
  for (int e = 1; e < EPT; ++e) tmax = fmaxf(tmax, v[e]);
  unsigned int tw = 0u;
  if (md.need_list) {
    const unsigned int k = f2key(tmax);
#pragma unroll 4
    for (int b = 31; b >= 0; --b) {
      const unsigned int c = tw | (1u << b);
      if (__popcll(__ballot(k >= c)) >= LIST / WAVES) tw = c;
    }
  }
  {
    const float wm = wave_max(tmax);
    if (lane == 0) {
      sh.rf[wid] = wm;
      sh.rint[wid] = static_cast<int>(tw);
    }
  }
  __syncthreads();  // B1
  float zmax = sh.rf[0];
#pragma unroll
  for (int w2 = 1; w2 < WAVES; ++w2) zmax = fmaxf(zmax, sh.rf[w2]);

  // ---- lowest index holding the max: only threads that hold it look.  Entries
  // at or past `end` read as -inf and come after the thread's valid entries.
  int targ = INT_MAX;
  if (tmax == zmax) {
#pragma unroll
    for (int e = EPT - 1; e >= 0; --e)
      if (v[e] == zmax && MLXF_IDX(e) < end) targ = MLXF_IDX(e);
  }

  // ---- log-sum-exp partial
  if (md.need_lse) {
    float t = 0.0f;
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if (MLXF_IDX(e) < end) t += wexp(v[e], zmax);
    const double ws = wave_sum(static_cast<double>(t));
    if (lane == 0) sh.rd[wid] = ws;
  }

  // ---- best-64 survivors.  theta, the smallest wave threshold, is reached by
  // at least 64 elements (16 thread maxima per wave), so the slice's best 64
  // all reach it.  Survivors are appended in LDS with one atomic per thread.
  if (md.need_list) {
    unsigned int tk = static_cast<unsigned int>(sh.rint[0]);
#pragma unroll
    for (int w2 = 1; w2 < WAVES; ++w2) tk = min(tk, static_cast<unsigned int>(sh.rint[w2]));
    const float thv = key2f(tk < KEY_NEG_INF ? KEY_NEG_INF : tk);
    if (tmax >= thv) {
      int mine = 0;
#pragma unroll
      for (int e = 0; e < EPT; ++e) mine += (v[e] >= thv && MLXF_IDX(e) < end) ? 1 : 0;
      if (mine > 0) {
        int pos = static_cast<int>(atomicAdd(&sh.ncand, static_cast<unsigned int>(mine)));
#pragma unroll
        for (int e = 0; e < EPT; ++e) {
          const int i = MLXF_IDX(e);
          if (v[e] >= thv && i < end) {
            if (pos < CAND_LDS) {
              r0.surv[pos].v = v[e];
              r0.surv[pos].i = i;
            }
            ++pos;
          }
        }
      }
    }
  }

  // ---- temperature-only / top-p: slice mass w = exp(z' - max z') and, for
  // top-p, the (count, truncated w) histogram of z' keys
  float mps = 0.0f;
  if (md.kind == KIND_TEMP || md.kind == KIND_TOPP) {
    mps = fz<DT>(zmax, md.Tr);
    const bool hist = md.kind == KIND_TOPP;
    double t = 0.0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      if (MLXF_IDX(e) < end) {
        const float zp = fz<DT>(v[e], md.Tr);
        const float w = wexp(zp, mps);
        t += static_cast<double>(w);
        if (hist)
          atomicAdd(&r1.hist[f2key(zp) >> 21],
                    (1ull << 40) +
                        static_cast<unsigned long long>(static_cast<unsigned int>(w * 16777216.0f)));
      }
    }
    const double ws = wave_sum(t);
    if (lane == 0) sh.rd2[wid] = ws;
  } else if (md.kind == KIND_KHIST) {
#pragma unroll
    for (int e = 0; e < EPT; ++e)
      if (MLXF_IDX(e) < end) atomicAdd(&r1.cnt[f2key(v[e]) >> 20], 1u);
  }
  {
    const int wa = wave_min(targ);
    if (lane == 0) sh.ri[wid] = wa;
  }
  __syncthreads();  // B2
  int zarg = sh.ri[0];
#pragma unroll
  for (int w2 = 1; w2 < WAVES; ++w2) zarg = min(zarg, sh.ri[w2]);
  double lse_s = 0.0, msum = 0.0;
  if (md.need_lse) {
    lse_s = sh.rd[0];
#pragma unroll
    for (int w2 = 1; w2 < WAVES; ++w2) lse_s += sh.rd[w2];
  }
  if (md.kind == KIND_TEMP || md.kind == KIND_TOPP) {
    msum = sh.rd2[0];
#pragma unroll
    for (int w2 = 1; w2 < WAVES; ++w2) msum += sh.rd2[w2];
  }

  // ---- best 64 of the slice from the survivors
  if (md.need_list) {
    int ntot = static_cast<int>(sh.ncand);
    if (ntot > CAND_LDS) {
      // Heavy ties at theta: the exact (value desc, index asc) 64th best thread
      // maximum instead, which at most 64 * EPT elements reach.
      int tbi = INT_MAX;
#pragma unroll
      for (int e = EPT - 1; e >= 0; --e)
        if (v[e] == tmax && MLXF_IDX(e) < end) tbi = MLXF_IDX(e);
      float lv = tmax;
      int li = tbi;
      wave_sort(lv, li);
      tree_merge(lv, li, sh.lists, WAVES);
      if (tid == LIST - 1) {
        sh.thv = lv;
        sh.thi = li;
      }
      __syncthreads();
      const float tv = sh.thv;
      const int ti = sh.thi;
      int mine = 0;
#pragma unroll
      for (int e = 0; e < EPT; ++e) mine += (MLXF_IDX(e) < end && !better(tv, ti, v[e], MLXF_IDX(e))) ? 1 : 0;
      int pos = block_excl_scan<int>(mine, sh.rint, &ntot);
#pragma unroll
      for (int e = 0; e < EPT; ++e) {
        const int i = MLXF_IDX(e);
        if (i < end && !better(tv, ti, v[e], i)) {
          r0.surv[pos].v = v[e];
          r0.surv[pos].i = i;
          ++pos;
        }
      }
      __syncthreads();
    }
    // 64-entry chunks: wave w sorts chunks w, w + WAVES, ... into its own list
    const int nch = (ntot + LIST - 1) / LIST;
    float sv = -INFINITY;
    int si = INT_MAX;
    for (int ch = wid; ch < nch; ch += WAVES) {
      const int c = ch * LIST + lane;
      float cv = -INFINITY;
      int ci = INT_MAX;
      if (c < ntot) {
        cv = r0.surv[c].v;
        ci = r0.surv[c].i;
      }
      wave_sort(cv, ci);
      wave_list_merge(sv, si, cv, ci);
    }
    tree_merge(sv, si, sh.lists, nch < WAVES ? nch : WAVES);
    if (wid == 0) st_dev(a.list + (static_cast<size_t>(r) * S + s) * LIST + lane, pack_ent(sv, si));
  }

  unsigned int ncand = 0;
  if (md.kind == KIND_TOPP) {
    const size_t off = (static_cast<size_t>(r) * S + s) * NBIN;
    for (int b = tid; b < NBIN; b += THREADS) st_dev(a.hist + off + b, r1.hist[b]);
  } else if (md.kind == KIND_KHIST) {
    // the bin of the slice's k-th largest z; thread t owns descending
    // positions PC*t .. PC*t+PC-1
    constexpr int PC = CNT_BINS / THREADS;
    int cq[PC], sumq = 0;
#pragma unroll
    for (int q = 0; q < PC; ++q) {
      cq[q] = static_cast<int>(r1.cnt[CNT_BINS - 1 - (PC * tid + q)]);
      sumq += cq[q];
    }
    int total;
    const int ex = block_excl_scan<int>(sumq, sh.rint, &total);
    const int kk_s = md.kk < (end - beg) ? md.kk : (end - beg);
    int run = ex;
#pragma unroll
    for (int q = 0; q < PC; ++q) {
      if (run < kk_s && run + cq[q] >= kk_s) sh.sel[0] = CNT_BINS - 1 - (PC * tid + q);
      run += cq[q];
    }
    __syncthreads();
    if (tid == 0) {
      const unsigned int edge = max(static_cast<unsigned int>(sh.sel[0]) << 20, KEY_NEG_INF);
      sh.sel[1] = static_cast<int>(gkey<DT>(fz<DT>(key2f(edge), md.Tr), md.Tr));
    }
    __syncthreads();
    const unsigned int thr = static_cast<unsigned int>(sh.sel[1]);
    int mine = 0;
#pragma unroll
    for (int e = 0; e < EPT; ++e) mine += (MLXF_IDX(e) < end && f2key(v[e]) >= thr) ? 1 : 0;
    int ctot;
    int pos = block_excl_scan<int>(mine, sh.rint, &ctot);
    uint2* dst = a.cand + (static_cast<size_t>(r) * S + s) * a.L;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      const int i = MLXF_IDX(e);
      const unsigned int key = f2key(v[e]);
      if (i < end && key >= thr) st_dev(dst + pos++, make_uint2(key, static_cast<unsigned int>(i)));
    }
    ncand = static_cast<unsigned int>(ctot);
  }
#undef MLXF_IDX

  if (tid == 0) {
    unsigned long long* rp = reinterpret_cast<unsigned long long*>(a.rec + (r * S + s));
    st_dev(rp + 0, pack2(__float_as_uint(zmax), static_cast<unsigned int>(zarg)));
    st_dev(rp + 1, pack2(__float_as_uint(mps), ncand));
    st_dev(rp + 2, static_cast<unsigned long long>(__double_as_longlong(lse_s)));
    st_dev(rp + 3, static_cast<unsigned long long>(__double_as_longlong(msum)));
  }

  // ---- ticket: the last slice of the row finishes it.  Every wave waits for
  // its device-coherent stores to complete before the ticket is drawn.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    sh.ticket = __hip_atomic_fetch_add(a.ctr + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (sh.ticket != static_cast<unsigned int>(S - 1)) return;
  if (tid == 0) {
    __hip_atomic_store(a.ctr + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next call
    sh.args = a;
    sh.md = md;
  }
  __syncthreads();
  finish_row<DT, EPT, VECOK>(r, r0, r1, sh);
}

// Zero the per-row counters of a fresh workspace.
__global__ void k_zero(unsigned int* p, size_t n) {
  const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// ================================================================ host side ==

struct Layout {
  int S, L, EPT;
  size_t off_ctr, off_rec, off_list, off_hist, off_cand, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

constexpr size_t CTR_BYTES_MAX = 65536 * sizeof(unsigned int);

// EPT: the largest of {32, 16, 8} that still gives at least one workgroup
// per CU (256) with at most MAX_S slices per row; otherwise the smallest EPT
// with S <= MAX_S (short batches: as many slices as allowed).
Layout make_layout(int B, int V, int K_max) {
  (void)K_max;
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
  size_t o = 0;
  l.off_ctr = o;  // first: mlxf_sampler_workspace_init zeroes the start of the buffer
  o = align256(o + sizeof(unsigned int) * (B > 0 ? B : 1));
  l.off_rec = o;
  o = align256(o + sizeof(SliceRec) * BS);
  l.off_list = o;
  o = align256(o + sizeof(unsigned long long) * BS * LIST);
  l.off_hist = o;
  o = align256(o + sizeof(unsigned long long) * BS * NBIN);
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

template <int DT, int EPT>
hipError_t launch_ept(const Args& a, bool vecok, hipStream_t st) {
  const dim3 grid(a.S, a.B);
  if (vecok)
    hipLaunchKernelGGL((k_sample<DT, EPT, true>), grid, dim3(THREADS), 0, st, a);
  else
    hipLaunchKernelGGL((k_sample<DT, EPT, false>), grid, dim3(THREADS), 0, st, a);
  return hipGetLastError();
}

template <int DT>
hipError_t launch_dt(const Args& a, int ept, bool vecok, hipStream_t st) {
  switch (ept) {
    case 8:
      return launch_ept<DT, 8>(a, vecok, st);
    case 16:
      return launch_ept<DT, 16>(a, vecok, st);
    default:
      return launch_ept<DT, 32>(a, vecok, st);
  }
}

int run_sample(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
               const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
               const int32_t* d_top_logprobs, const float* d_uniforms, int32_t* d_out_ids,
               float* d_out_logprobs, int32_t* d_out_top_ids, float* d_out_top_logprobs,
               int K_max, void* d_workspace, size_t workspace_bytes, void* stream, char** err) {
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
    a.ctr = reinterpret_cast<unsigned int*>(ws + l.off_ctr);
    a.rec = reinterpret_cast<SliceRec*>(ws + l.off_rec);
    a.list = reinterpret_cast<unsigned long long*>(ws + l.off_list);
    a.hist = reinterpret_cast<unsigned long long*>(ws + l.off_hist);
    a.cand = reinterpret_cast<uint2*>(ws + l.off_cand);
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e;
    if (dtype == MLXF_DTYPE_F32)
      e = launch_dt<MLXF_DTYPE_F32>(a, l.EPT, vecok, st);
    else if (dtype == MLXF_DTYPE_BF16)
      e = launch_dt<MLXF_DTYPE_BF16>(a, l.EPT, vecok, st);
    else
      e = launch_dt<MLXF_DTYPE_F16>(a, l.EPT, vecok, st);
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
    *bytes = make_layout(B, V, K_max).total;
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
  return run_sample(d_logits, dtype, B, V, row_stride, d_temperature, d_top_k, d_top_p,
                    d_top_logprobs, d_uniforms, d_out_ids, d_out_logprobs, d_out_top_ids,
                    d_out_top_logprobs, K_max, d_workspace, workspace_bytes, stream, err);
}

int mlxf_greedy(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                int32_t* d_out_ids, void* d_workspace, size_t workspace_bytes, void* stream,
                char** err) {
  return run_sample(d_logits, dtype, B, V, row_stride, nullptr, nullptr, nullptr, nullptr, nullptr,
                    d_out_ids, nullptr, nullptr, nullptr, 0, d_workspace, workspace_bytes, stream,
                    err);
}

}  // extern "C"
