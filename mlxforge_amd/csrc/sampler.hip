// sampler.hip -- MI355X (gfx950) batched token sampler behind the C ABI in
// include/mlxf_sampler.h.
//
// Replaces the per-row MLX graph of Sampler::sample (src/sample/sampler.cpp:
// 141-166), run once per row by Worker::sample_rows (src/runtime/worker.cpp:
// 448-486), with ONE kernel launch over all rows of a [B, V] logits matrix.
//
// One launch, a 1-D grid of B * S first-pass workgroups followed by up to 256
// helper workgroups.  Row r is cut into S slices of L = 256 * EPT elements
// (EPT in {8, 16, 32}); slice s is workgroup r * S + s (256 threads, 4 waves,
// up to 256 VGPRs each, two workgroups per CU), which loads its whole slice
// into registers with 16-byte loads (the one HBM read of the logits) and
// reduces it there:
//   * max and lowest-index argmax of z, and sum exp(z - max) when a logprob is
//     wanted;
//   * when top_logprobs or a top-k <= 63 is asked for: the slice's best 64
//     entries by (z desc, index asc).  The 64th best of the 256 per-thread
//     maxima bounds the slice's 64th best from below; the at most 64 * EPT
//     elements at or above it are sorted in 64-entry chunks and merged;
//   * top-k > 63: a 4096-bin count histogram of z keys (the bins the slice
//     occupies are recorded);
//   * temperature-only and top-p rows: the sum of w = exp(z' - max z') over the
//     slice (z' = z / T in the logits dtype), and for top-p a 2048-bin
//     histogram of z' keys holding (count, exact 2^-42 fixed-point mass).
// The slice then takes a ticket on the row's counter; the workgroup that draws
// the row's last ticket finishes the row:
//   * greedy: argmax, logprob and top_logprobs from the slice summaries;
//   * top-k <= 63: the merged best-64 list of the row decides everything in one
//     wave (the k-th largest z', the nucleus prefix, the draw), after checking
//     that the list holds every element at or above the k-th value of z';
//   * temperature-only: the slice that holds u * sum(w), then a walk of that
//     slice in vocabulary order;
//   * top-p and top-k > 63: the combined histograms bracket the cutoff in a
//     narrow range of z' values, and the finisher writes a plan for a second
//     pass and queues the row.
// Second pass: one item per slice of a queued row, taken by the row's finisher
// or by the helper workgroups (which poll the queue until every row of the
// call is done).  An item re-reads its slice and keeps only what lies in the
// bracket: per-value counts and masses when the bracket holds few distinct
// 16-bit values, else the candidates themselves.  The row's last item resolves
// the cutoff (the value, and the last kept index among its ties), the kept
// mass, and the draw (the one slice holding u * kept mass, walked in
// vocabulary order).  Nothing ever waits for a workgroup that may not have
// started: the ticket holder does the work, and helpers only take queued work.
// Masses that decide a cutoff are exact 64-bit fixed-point sums (2^-42 units)
// or fp64 sums in a fixed order, so every result is reproducible bit for bit.
// Data one workgroup leaves for another travels through device-coherent (sc1)
// loads and stores, so no L2-wide write-back is ever needed.
// Counters that must read zero at the start of a call are either reset by
// their last user or stamped with a per-call epoch.
// There is no MFMA anywhere: nothing here is a dense contraction.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>
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
  unsigned int* ctr;          // [B] first-pass tickets
  unsigned int* done2;        // [B] second-pass tickets
  unsigned long long* next2;  // [B] second-pass items taken (epoch-stamped)
  unsigned long long* gl;     // call-wide counters (GL_*, epoch-stamped)
  unsigned long long* queue;  // [B] rows with second-pass items: (epoch, row + 1)
  unsigned int epoch;         // this call's stamp (never 0)
  int helpers;                // workgroups after the first B*S
  SliceRec* rec;
  unsigned long long* list;   // [B*S][64] packed (z bits, index)
  unsigned long long* hist;   // [B*S][NBIN]
  uint2* cand;                // [B*S][L]
  unsigned long long* plan;   // [B][PLAN_WORDS]
  double* above;              // [B*S] mass above the bracket, slice units
  unsigned int* ncand2;       // [B*S] second-pass candidates per slice
};

// Call-wide counters: queue slots reserved, rows finished, whether any row of
// the call has a second pass, and the first queue slot whose row may still have
// items left.  These, the per-row item counters and the
// queue slots are 64-bit words (epoch << 32 | value): a word stamped by another
// call reads as zero, so nothing needs resetting between calls.  (The per-row
// tickets ctr / done2 are plain counters, reset by their last user.)
enum { GL_QRES = 0, GL_ROWS = 1, GL_NEED = 2, GL_HEAD = 3, GL_WORDS = 8 };
constexpr int IDLE_LIMIT = 1 << 16;  // bound on a helper's idle polls (each sleeps up to ~2 us)

__device__ __forceinline__ unsigned int stamped(unsigned long long w, unsigned int epoch) {
  return static_cast<unsigned int>(w >> 32) == epoch ? static_cast<unsigned int>(w) : 0u;
}
__device__ __forceinline__ unsigned int stamped_get(const unsigned long long* p, unsigned int epoch) {
  return stamped(ld_dev(p), epoch);
}
// Take the next value of a stamped counter: the first taker in a call claims
// the word (compare-exchange from the stale stamp to (epoch, 1)), everyone
// else adds 1.  Returns the value taken, or `limit` once it has reached limit
// (the low half never reaches the stamp: there are far fewer takers than 2^32).
__device__ __forceinline__ unsigned int stamped_take(unsigned long long* p, unsigned int epoch,
                                                     unsigned int limit) {
  unsigned long long w = ld_dev(p);
  if (static_cast<unsigned int>(w >> 32) != epoch) {
    const unsigned long long claim = (static_cast<unsigned long long>(epoch) << 32) | 1u;
    if (__hip_atomic_compare_exchange_strong(p, &w, claim, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT))
      return 0u < limit ? 0u : limit;
    if (static_cast<unsigned int>(w >> 32) != epoch) return limit;  // (another call's stamp: not ours)
  }
  const unsigned long long old = __hip_atomic_fetch_add(p, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  const unsigned int v = static_cast<unsigned int>(old);
  return v < limit ? v : limit;
}

// The plan a row's first pass leaves for its second pass (64-bit words): bracket z-key range [klo, khi), has_hi, value
// mode (nv > 0: nv z' values from value index vbase), the nucleus mass still to
// cover inside the bracket (2^-42 row units), the row's LSE and max z'.
enum { PL_KEYS = 0, PL_MODE = 1, PL_TARGET = 2, PL_LSE = 3, PL_MP = 4, PLAN_WORDS = 5 };

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
  unsigned int vcnt[2 * CAND_LDS];     // 16-bit counters, two per word
  unsigned short vc16[4 * CAND_LDS];   // per (slice, z' value) counts
  TopEnt surv[CAND_LDS];  // >= 64 * EPT: the most elements that can reach theta
};
union Region1 {  // 16 KB
  unsigned int cnt[CNT_BINS];
  unsigned long long hist[NBIN];  // exact 2^-42 masses of w(z', mps) per z'-key bin
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
  int bmin[WAVES], bmax[WAVES];
  int rlo[MAX_S], rhi[MAX_S];  // occupied histogram bins per slice
  unsigned long long plan[PLAN_WORDS];
  int qrow, qitem;
  unsigned int qn, rdone;
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

// z' value index shift for the 16-bit types: z' is a bf16 / f16 value held in
// fp32, so its key's low VSHIFT bits carry no information.
template <int DT>
constexpr int vshift() {
  return DT == MLXF_DTYPE_BF16 ? 16 : 13;
}

// Compare-only pass over the row (the finishing workgroup alone).  Elements
// with z key in [klo, khi) are "in range"; their mass (2^-42 units of
// w(z', mps_t)) goes to r1.pass.sq[t * WAVES + wave].  In candidate mode
// (nv == 0) they become candidates (z' key, index); in value mode (nv > 0, the
// 16-bit types) they are counted per (slice, z' value) in 16-bit counters
// r0.vcnt (value index (z' key >> vshift) - vbase).  When `sum_side` is 1
// (above: z key >= khi) or 2 (below: z key < klo) the mass of that side goes to
// r1.pass.sp (fp64).  has_hi false: no upper bound.  The next slice's loads
// are in flight while a slice is processed.
template <int DT, int EPT, bool VECOK>
__device__ void row_pass(const Args& a, const Mode& md, const void* row, int r, unsigned int klo,
                         bool has_hi, unsigned int khi, int sum_side, int nv, unsigned int vbase,
                         Region0& r0, Region1& r1, Small& sh) {
  constexpr int NIT = EPT / VEC;
  const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
  const int S = a.S;
  uint2* g = a.cand + static_cast<size_t>(r) * S * a.L;
  if (nv > 0) {
    for (int w = tid; w < (S * nv + 1) / 2; w += THREADS) r0.vcnt[w] = 0u;
    __syncthreads();
  }
  // double buffer: slice t+1's loads are in flight while slice t is processed
  Raw8<DT> cur[NIT], nxt[NIT];
#pragma unroll
  for (int it = 0; it < NIT; ++it) load_raw<DT, VECOK>(row, it * CHUNK + tid * VEC, min(a.V, a.L), cur[it]);
#pragma unroll 1
  for (int t = 0; t < S; ++t) {
    const int b0 = t * a.L, e0 = min(a.V, b0 + a.L);
    if (t + 1 < S) {
      const int nb0 = b0 + a.L, ne0 = min(a.V, nb0 + a.L);
#pragma unroll
      for (int it = 0; it < NIT; ++it) load_raw<DT, VECOK>(row, nb0 + it * CHUNK + tid * VEC, ne0, nxt[it]);
    }
    const float mps = sh.mps[t];
    double part = 0.0;
    unsigned long long pq = 0;
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      float z[VEC];
      decode8<DT>(cur[it], z);
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
          if (side) part += static_cast<double>(w);
          if (inr) pq += quant(w);
          zpk = f2key(zp);
        }
        if (nv > 0) {
          if (inr) {
            const unsigned int c = static_cast<unsigned int>(t * nv) + ((zpk >> vshift<DT>()) - vbase);
            atomicAdd(&r0.vcnt[c >> 1], 1u << (16 * (c & 1u)));
          }
        } else {
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
    }
    const double pd = wave_sum(part);
    pq = wave_sum(pq);
    if (lane == 0) {
      r1.pass.sp[t * WAVES + wid] = pd;
      r1.pass.sq[t * WAVES + wid] = pq;
    }
#pragma unroll
    for (int it = 0; it < NIT; ++it) cur[it] = nxt[it];
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
    row_pass<DT, EPT, VECOK>(a, md, row, r, static_cast<unsigned int>(sh.sel[4]), false, 0u, 0, 0, 0u,
                             r0, r1, sh);
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

// Top-p without top-k, end of the first pass (the row's last slice): combine the
// slices' exact mass histograms (occupied bins only) in row units, bracket the
// nucleus boundary -- the bins [blo, bhi] whose cumulative mass from the top
// reaches p * W within a relative 1e-12 -- and leave the plan for the second
// pass: the bracket as z-key thresholds (no division in the comparisons),
// value mode when the logits are 16-bit and the bracket holds few z' values,
// p * W, the LSE and max z'; then queue the row for its second pass, whose S
// items (one per slice) any workgroup may take.  Thread t owns descending
// positions PB*t ..
// PB*t+PB-1, i.e. the consecutive bins hb0 .. hb0+PB-1 (position PB*t+q is bin
// hb0+PB-1-q); four slices' histograms are read per round.
template <int DT>
__device__ void plan_topp(const Args& a, const Mode& md, int r, Small& sh) {
  const int tid = threadIdx.x;
  const int S = a.S;
  constexpr int PB = NBIN / THREADS;
  if (tid < S) {
    const unsigned int rg = sh.ncnd[tid];
    sh.rlo[tid] = static_cast<int>(rg & 0xffffu);
    sh.rhi[tid] = static_cast<int>(rg >> 16);
  }
  if (tid == 0) {
    sh.pos_hi = NBIN;
    sh.pos_lo = NBIN;
    sh.pos_last = -1;
  }
  __syncthreads();
  const unsigned long long* hrow = a.hist + static_cast<size_t>(r) * S * NBIN;
  const int hb0 = NBIN - PB * (tid + 1);
  double m[PB];
#pragma unroll
  for (int q = 0; q < PB; ++q) m[q] = 0.0;
#pragma unroll 1
  for (int t0 = 0; t0 < S; t0 += 4) {
    unsigned long long h[4][PB];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int t = t0 + u;
      const int lo = t < S ? sh.rlo[t] : NBIN, hi = t < S ? sh.rhi[t] : -1;
#pragma unroll
      for (int j = 0; j < PB; ++j) {
        const int b = hb0 + j;
        h[u][j] = (b >= lo && b <= hi) ? ld_dev(hrow + static_cast<size_t>(t) * NBIN + b) : 0ull;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const double sc = t0 + u < S ? sh.scale[t0 + u] * QUNIT : 0.0;
#pragma unroll
      for (int j = 0; j < PB; ++j) m[PB - 1 - j] += static_cast<double>(h[u][j]) * sc;
    }
  }
  double sA = 0.0;
#pragma unroll
  for (int q = 0; q < PB; ++q) sA += m[q];
  double exA, inA, W;
  block_scan<double>(sA, sh.rd, &exA, &inA, &W);
  const double PW = static_cast<double>(md.pr) * W;
  const double t_hi = PW * (1.0 - 1e-12), t_lo = PW * (1.0 + 1e-12);
  int ph = NBIN, pl = NBIN, last = -1;
  double run = exA;
#pragma unroll
  for (int q = 0; q < PB; ++q) {
    run += m[q];
    if (m[q] > 0.0) {
      if (ph == NBIN && run >= t_hi) ph = PB * tid + q;
      if (pl == NBIN && run >= t_lo) pl = PB * tid + q;
      last = PB * tid + q;
    }
  }
  if (ph < NBIN) atomicMin(&sh.pos_hi, ph);
  if (pl < NBIN) atomicMin(&sh.pos_lo, pl);
  if (last >= 0) atomicMax(&sh.pos_last, last);
  __syncthreads();
  if (tid == 0) {
    const int p_last = sh.pos_last < 0 ? NBIN - 1 : sh.pos_last;
    const int p_hi = min(sh.pos_hi, p_last), p_lo = min(sh.pos_lo, p_last);
    const int bhi = NBIN - 1 - p_hi, blo = NBIN - 1 - p_lo;
    const unsigned int klo_edge = max(static_cast<unsigned int>(blo) << 21, KEY_NEG_INF);
    const unsigned int klo = gkey<DT>(key2f(klo_edge), md.Tr);
    const unsigned int hi_edge = static_cast<unsigned int>(bhi + 1) << 21;
    const bool has_hi = bhi < NBIN - 1 && hi_edge <= KEY_POS_INF;
    const unsigned int khi = has_hi ? gkey<DT>(key2f(hi_edge), md.Tr) : 0u;
    // value mode: every z' in the bracket is one of nv 16-bit values, counted
    // per (slice, value) in 16-bit LDS counters by the resolving workgroup
    int nv = 0;
    if (DT != MLXF_DTYPE_F32) {
      const int vpb = 1 << (21 - vshift<DT>());
      const int want = (bhi - blo + 1) * vpb;
      if (want <= 1024 && want * S <= 4 * CAND_LDS) nv = want;
    }
    const unsigned int vbase = static_cast<unsigned int>(blo) << (21 - vshift<DT>());
    unsigned long long* pl_ = a.plan + static_cast<size_t>(r) * PLAN_WORDS;
    st_dev(pl_ + PL_KEYS, pack2(klo, khi));
    st_dev(pl_ + PL_MODE, pack2(static_cast<unsigned int>(has_hi ? 1 : 0) | (static_cast<unsigned int>(bhi) << 1),
                                static_cast<unsigned int>(nv) | (vbase << 11)));  // kind bit 12 clear: top-p
    st_dev(pl_ + PL_TARGET, static_cast<unsigned long long>(__double_as_longlong(PW)));
    st_dev(pl_ + PL_LSE, static_cast<unsigned long long>(__double_as_longlong(sh.lse)));
    st_dev(pl_ + PL_MP, static_cast<unsigned long long>(__float_as_uint(sh.Mp)));
    __builtin_amdgcn_s_waitcnt(0);  // the plan is complete before the row is queued
    const unsigned int qp = stamped_take(a.gl + GL_QRES, a.epoch, 0xffffffffu);
    st_dev(a.queue + qp, (static_cast<unsigned long long>(a.epoch) << 32) | (static_cast<unsigned int>(r) + 1u));
  }
}

// Top-k with k > 63, end of the first pass: the z-key bin that holds the
// row's k-th largest z, from the slices' count histograms (occupied bins only);
// the plan's bracket is every element whose z' reaches the z' of that bin's
// lower edge (z key >= klo, no upper bound).  Value mode when the logits are
// 16-bit and few z' values lie between that edge and the row's max z'.  Then
// queue the row for its second pass.  Thread t owns descending positions
// PC*t .. PC*t+PC-1 (bins cb0 .. cb0+PC-1).
template <int DT>
__device__ void plan_topk(const Args& a, const Mode& md, int r, Small& sh) {
  const int tid = threadIdx.x;
  const int S = a.S;
  constexpr int PC = CNT_BINS / THREADS;
  if (tid < S) {
    const unsigned int rg = sh.ncnd[tid];
    sh.rlo[tid] = static_cast<int>(rg & 0xffffu);
    sh.rhi[tid] = static_cast<int>(rg >> 16);
  }
  if (tid == 0) sh.pos_hi = CNT_BINS;
  __syncthreads();
  const unsigned int* hrow = reinterpret_cast<const unsigned int*>(a.hist + static_cast<size_t>(r) * S * NBIN);
  const int cb0 = CNT_BINS - PC * (tid + 1);
  unsigned int c[PC];
#pragma unroll
  for (int q = 0; q < PC; ++q) c[q] = 0u;
#pragma unroll 1
  for (int t0 = 0; t0 < S; t0 += 2) {
    unsigned int h[2][PC];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = t0 + u;
      const int lo = t < S ? sh.rlo[t] : CNT_BINS, hi = t < S ? sh.rhi[t] : -1;
#pragma unroll
      for (int j = 0; j < PC; ++j) {
        const int b = cb0 + j;
        h[u][j] = (b >= lo && b <= hi)
                      ? __hip_atomic_load(hrow + static_cast<size_t>(t) * CNT_BINS + b, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT)
                      : 0u;
      }
    }
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int j = 0; j < PC; ++j) c[PC - 1 - j] += h[u][j];
  }
  unsigned int sum = 0;
#pragma unroll
  for (int q = 0; q < PC; ++q) sum += c[q];
  unsigned int ex, in, tot;
  block_scan<unsigned int>(sum, reinterpret_cast<unsigned int*>(sh.rint), &ex, &in, &tot);
  const unsigned int kk = static_cast<unsigned int>(md.kk);
  unsigned int run = ex;
  int found = CNT_BINS;
#pragma unroll
  for (int q = 0; q < PC; ++q) {
    if (found == CNT_BINS && c[q] > 0 && run + c[q] >= kk) found = PC * tid + q;
    run += c[q];
  }
  if (found < CNT_BINS) atomicMin(&sh.pos_hi, found);
  __syncthreads();
  if (tid == 0) {
    const int pos = sh.pos_hi < CNT_BINS ? sh.pos_hi : CNT_BINS - 1;  // (k <= V: always found)
    const int bstar = CNT_BINS - 1 - pos;
    const unsigned int edge = max(static_cast<unsigned int>(bstar) << 20, KEY_NEG_INF);
    const unsigned int klo = gkey<DT>(fz<DT>(key2f(edge), md.Tr), md.Tr);
    int nv = 0;
    unsigned int vbase = 0;
    if (DT != MLXF_DTYPE_F32) {
      const unsigned int vlo = f2key(fz<DT>(key2f(klo), md.Tr)) >> vshift<DT>();
      const unsigned int vhi = f2key(sh.Mp) >> vshift<DT>();
      const int want = static_cast<int>(vhi - vlo + 2) & ~1;  // whole pairs of counters
      if (vhi >= vlo && want <= 1024 && want * S <= 4 * CAND_LDS) {
        nv = want;
        vbase = vlo;
      }
    }
    unsigned long long* pl_ = a.plan + static_cast<size_t>(r) * PLAN_WORDS;
    st_dev(pl_ + PL_KEYS, pack2(klo, 0u));
    st_dev(pl_ + PL_MODE, pack2(static_cast<unsigned int>(NBIN - 1) << 1 | (1u << 12),  // kind bit: top-k
                                static_cast<unsigned int>(nv) | (vbase << 11)));
    st_dev(pl_ + PL_TARGET, static_cast<unsigned long long>(kk));
    st_dev(pl_ + PL_LSE, static_cast<unsigned long long>(__double_as_longlong(sh.lse)));
    st_dev(pl_ + PL_MP, static_cast<unsigned long long>(__float_as_uint(sh.Mp)));
    __builtin_amdgcn_s_waitcnt(0);  // the plan is complete before the row is queued
    const unsigned int qp = stamped_take(a.gl + GL_QRES, a.epoch, 0xffffffffu);
    st_dev(a.queue + qp, (static_cast<unsigned long long>(a.epoch) << 32) | (static_cast<unsigned int>(r) + 1u));
  }
}

// Second pass, the row's last item: the exact nucleus cutoff inside the
// bracket and the draw.  Value mode (16-bit logits): per (slice, z' value)
// counts give the cutoff value v*, the number t of its ties that are kept
// (lowest indices first), the slice holding the t-th tie (scanned for its
// index) and every slice's kept mass.  Candidate mode: radix selections over
// the bracket's elements.  Then the slice that holds the draw is walked.
template <int DT, int EPT, bool VECOK>
__device__ void resolve_row(int r, Region0& r0, Region1& r1, Small& sh) {
  const Args& a = sh.args;
  const Mode& md = sh.md;
  const void* row = row_ptr<DT>(a, r);
  const int tid = threadIdx.x;
  const int S = a.S;
  const unsigned long long wmode = sh.plan[PL_MODE];
  const bool khist = ((wmode >> 12) & 1ull) != 0;  // top-k (k > 63) row, else top-p
  const int nv = static_cast<int>((wmode >> 32) & 0x7ffu);
  const unsigned int vbase = static_cast<unsigned int>(wmode >> 43);
  const double PW = khist ? 0.0 : __longlong_as_double(static_cast<long long>(sh.plan[PL_TARGET]));
  const unsigned int kk = khist ? static_cast<unsigned int>(sh.plan[PL_TARGET]) : 0u;
  const float Mp = __uint_as_float(static_cast<unsigned int>(sh.plan[PL_MP]));
  if (tid == 0) {
    sh.lse = __longlong_as_double(static_cast<long long>(sh.plan[PL_LSE]));
    sh.Mp = Mp;
  }
  if (tid < S) {
    const unsigned long long* rp = reinterpret_cast<const unsigned long long*>(a.rec + (r * S + tid));
    const float mps = __uint_as_float(static_cast<unsigned int>(ld_dev(rp + 1)));
    sh.mps[tid] = mps;
    sh.scale[tid] = wexp_d(mps, Mp);
    sh.keep[tid] = __longlong_as_double(static_cast<long long>(ld_dev(a.above + (r * S + tid))));
    sh.keepq[tid] = 0ull;
    sh.ncnd[tid] = nv > 0 ? 0u : __hip_atomic_load(a.ncand2 + (r * S + tid), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  if (tid == 0) {
    double pa = 0.0;
    for (int t = 0; t < S; ++t) pa += sh.keep[t] * sh.scale[t];
    const double nq = (PW - pa) / QUNIT;  // nucleus mass still to cover inside the bracket
    sh.selu[1] = nq <= 1.0 ? 1ull : static_cast<unsigned long long>(ceil(nq));
    int o = 0;
    for (int t = 0; t < S; ++t) {
      sh.off[t] = o;
      o += static_cast<int>(sh.ncnd[t]);
    }
    sh.off[S] = o;
  }
  __syncthreads();
  unsigned long long target = sh.selu[1];
  unsigned int vkey;
  int idx_cut = INT_MAX;
  if (nv > 0) {
    // per (slice, value) counts: slice t left nv/2 words of two 32-bit counts
    const int words = nv / 2;
#pragma unroll 4
    for (int idx = tid; idx < S * words; idx += THREADS) {
      const int t = idx / words, w = idx - t * words;
      const unsigned long long x =
          ld_dev(reinterpret_cast<const unsigned long long*>(a.cand + (static_cast<size_t>(r) * S + t) * a.L) + w);
      r0.vc16[t * nv + 2 * w] = static_cast<unsigned short>(x);
      r0.vc16[t * nv + 2 * w + 1] = static_cast<unsigned short>(x >> 32);
    }
    __syncthreads();
    // Values are scanned from the top (value index nv-1) down; thread t owns
    // descending positions 4t .. 4t+3.
    constexpr int VS = vshift<DT>();
    auto vkey_of = [vbase](int v) {
      const unsigned int top = vbase + static_cast<unsigned int>(v);
      return (top << VS) | (top < (0x80000000u >> VS) ? ((1u << VS) - 1u) : 0u);
    };
    auto cnt_of = [&](int t, int v) { return static_cast<unsigned int>(r0.vc16[t * nv + v]); };
    unsigned int cv[4];
    unsigned long long mv[4], msum4 = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos = 4 * tid + j, v = nv - 1 - pos;
      unsigned int cnt = 0;
      if (pos < nv)
        for (int t = 0; t < S; ++t) cnt += cnt_of(t, v);
      cv[j] = cnt;
      mv[j] = cnt ? static_cast<unsigned long long>(cnt) * quant(wexp(key2f(vkey_of(v)), Mp)) : 0ull;
      msum4 += mv[j];
    }
    if (tid == 0) {
      sh.pos_hi = nv;
      sh.pos_lo = nv;
      sh.pos_last = -1;
    }
    // top-k rows: the k-th largest z' (position plim, counted from the top),
    // the mass W_k of the values at or above it, and the nucleus target inside
    // them (all of W_k when there is no top-p)
    int plim = nv - 1;
    if (khist) {
      unsigned int csum = cv[0] + cv[1] + cv[2] + cv[3];
      unsigned int cex, cin, ctot;
      block_scan<unsigned int>(csum, reinterpret_cast<unsigned int*>(sh.rint), &cex, &cin, &ctot);
      unsigned int crun = cex;
      int fpos = nv;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (fpos == nv && cv[j] > 0 && crun + cv[j] >= kk) fpos = 4 * tid + j;
        crun += cv[j];
      }
      if (fpos < nv) atomicMin(&sh.pos_lo, fpos);
      __syncthreads();
      plim = sh.pos_lo < nv ? sh.pos_lo : nv - 1;
      unsigned long long part = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) part += (4 * tid + j <= plim) ? mv[j] : 0ull;
      const unsigned long long wk = block_sum<unsigned long long>(part, sh.ru);
      target = md.topp ? static_cast<unsigned long long>(ceil(static_cast<double>(md.pr) * static_cast<double>(wk)))
                       : wk;
      if (target == 0) target = 1;
    }
    unsigned long long ex, in, tot;
    block_scan<unsigned long long>(msum4, sh.ru, &ex, &in, &tot);
    unsigned long long run = ex;
    int found = nv, lastne = -1;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int pos = 4 * tid + j;
      if (cv[j] > 0 && pos <= plim) {
        if (found == nv && mv[j] > 0 && run + mv[j] >= target) found = pos;
        lastne = pos;
      }
      run += mv[j];
    }
    if (found < nv) atomicMin(&sh.pos_hi, found);
    if (lastne >= 0) atomicMax(&sh.pos_last, lastne);
    __syncthreads();
    // the position of v* and the mass of the values above it; a top-k row
    // without top-p keeps every tie of its k-th value
    const bool whole = khist && !md.topp;
    const int pstar = whole ? plim : (sh.pos_hi < nv ? sh.pos_hi : (sh.pos_last < 0 ? 0 : sh.pos_last));
    if (pstar >= 4 * tid && pstar < 4 * tid + 4) {
      unsigned long long pgt = ex;
      for (int j = 0; j < pstar - 4 * tid; ++j) pgt += mv[j];
      const int jj = pstar - 4 * tid;
      const unsigned int cstar = cv[jj];
      const unsigned long long wstar = cstar ? mv[jj] / cstar : 0ull;
      unsigned long long t = cstar;
      if (!whole && sh.pos_hi < nv && wstar > 0) {
        const unsigned long long nd = target > pgt ? (target - pgt + wstar - 1) / wstar : 0ull;
        t = nd < t ? nd : t;
      }
      if (t == 0) t = 1;
      sh.selu[2] = t;
      sh.sel[14] = static_cast<int>(cstar);
    }
    __syncthreads();
    const int vstar = nv - 1 - pstar;
    vkey = vkey_of(vstar);
    const unsigned int tties = static_cast<unsigned int>(sh.selu[2]);
    const unsigned int cstar = static_cast<unsigned int>(sh.sel[14]);
    if (tid == 0) {  // the slice holding the t-th tie and its rank there
      unsigned int before = 0;
      int st = S - 1;
      for (int t = 0; t < S; ++t) {
        const unsigned int ct = cnt_of(t, vstar);
        if (before + ct >= tties) {
          st = t;
          break;
        }
        before += ct;
      }
      sh.sel[15] = st;
      sh.selu[3] = tties - before;
    }
    __syncthreads();
    const int st_tie = sh.sel[15];
    const unsigned int rank = static_cast<unsigned int>(sh.selu[3]);
    if (tties < cstar) {
      // index of the rank-th element equal to v* in slice st_tie (thread t owns
      // EPT consecutive elements)
      const int b0 = st_tie * a.L, e0 = min(a.V, b0 + a.L);
      const int my0 = b0 + tid * EPT;
      unsigned int cnt = 0;
#pragma unroll 2
      for (int it = 0; it < EPT / VEC; ++it) {
        float z[VEC];
        load8<DT, VECOK>(row, my0 + it * VEC, e0, z);
#pragma unroll
        for (int j = 0; j < VEC; ++j)
          cnt += (my0 + it * VEC + j < e0 && f2key(fz<DT>(z[j], md.Tr)) == vkey) ? 1u : 0u;
      }
      unsigned int cex, cin, ctot;
      block_scan<unsigned int>(cnt, reinterpret_cast<unsigned int*>(sh.rint), &cex, &cin, &ctot);
      if (cex < rank && rank <= cin) {
        unsigned int k = cex;
        int pick = -1;
        for (int it = 0; it < EPT / VEC && pick < 0; ++it) {
          float z[VEC];
          load8<DT, VECOK>(row, my0 + it * VEC, e0, z);
#pragma unroll
          for (int j = 0; j < VEC; ++j) {
            const int i = my0 + it * VEC + j;
            if (pick < 0 && i < e0 && f2key(fz<DT>(z[j], md.Tr)) == vkey && ++k == rank) pick = i;
          }
        }
        sh.sel[1] = pick;
      }
      __syncthreads();
      idx_cut = sh.sel[1];
    }
    // kept in-bracket mass per slice: values above v*, and the ties up to the cut
    for (int pidx = tid; pidx < S * nv; pidx += THREADS) {
      const int t = pidx / nv, v = pidx - t * nv;
      unsigned long long q = 0;
      if (v >= vstar) {
        unsigned int cnt = cnt_of(t, v);
        if (v == vstar && tties < cstar) cnt = t < st_tie ? cnt : (t == st_tie ? rank : 0u);
        if (cnt) q = static_cast<unsigned long long>(cnt) * quant(wexp(key2f(vkey_of(v)), sh.mps[t]));
      }
      if (q) atomicAdd(&sh.keepq[t], q);
    }
    __syncthreads();
  } else {
    // candidate mode: the bracket's elements, per-slice regions of a.cand
    const int n = sh.off[S];
    CandView cv;
    cv.l = nullptr;
    cv.g = a.cand + static_cast<size_t>(r) * S * a.L;
    cv.off = sh.off;
    cv.S = S;
    cv.L = a.L;
    if (n <= CAND_LDS) {  // gather into LDS
      for (int t = 0; t < S; ++t) {
        const int o = sh.off[t], cnt = sh.off[t + 1] - o;
        const uint2* src = cv.g + static_cast<size_t>(t) * a.L;
        for (int j = tid; j < cnt; j += THREADS) r0.cand[o + j] = ld_dev2(src + j);
      }
      __syncthreads();
      cv.l = r0.cand;
    }
    if (khist) {  // k-th largest, top-p inside the top k, and the draw, on the candidates
      const int id = resolve_topk(md, cv, n, Mp, sh);
      write_sampled<DT>(a, md, row, r, id, sh);
      if (tid == 0) stamped_take(a.gl + GL_ROWS, a.epoch, 0xffffffffu);
      return;
    }
    auto wq = [Mp](uint2 e) { return quant(wexp(key2f(e.x), Mp)); };
    unsigned long long pgt, bef;
    unsigned int g_cnt;
    bool all_kept;
    auto any = [](uint2) { return true; };
    vkey = radix_select<true, true, true>(cv, n, any, wq, target, false, sh, &pgt, &g_cnt, &all_kept);
    const unsigned long long wstar = wq(make_uint2(vkey, 0u));
    unsigned long long tk = g_cnt;
    if (!all_kept && wstar > 0) {
      const unsigned long long nd = target > pgt ? (target - pgt + wstar - 1) / wstar : 0ull;
      tk = nd < tk ? nd : tk;
    }
    if (tk == 0) tk = 1;
    if (tk < g_cnt) {
      const unsigned int vk = vkey;
      auto eq_v = [vk](uint2 e) { return e.x == vk; };
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
  }
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
  if (tid == 0) stamped_take(a.gl + GL_ROWS, a.epoch, 0xffffffffu);
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
    plan_topk<DT>(a, md, r, sh);
    return;  // finished by its second pass
  } else if (md.kind == KIND_TOPP) {
    plan_topp<DT>(a, md, r, sh);
    return;  // finished by its second pass
  }
  if (tid == 0) stamped_take(a.gl + GL_ROWS, a.epoch, 0xffffffffu);
}

// =================================================================== kernel ==

// First pass over slice s of row r; the row's last slice finishes the row
// (returns true in that workgroup).
template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ bool first_pass(const Args& a, int r, int s, Region0& r0, Region1& r1, Small& sh) {
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
  if (s == 0 && tid == 0 && (md.kind == KIND_TOPP || md.kind == KIND_KHIST))
    st_dev(a.gl + GL_NEED, (static_cast<unsigned long long>(a.epoch) << 32) | 1u);

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
  // top-p, the exact (2^-42 units) mass histogram of z' keys with the range of
  // occupied bins
  const float mps = md.sampling ? fz<DT>(zmax, md.Tr) : 0.0f;  // the slice's weight reference
  if (md.kind == KIND_TEMP || md.kind == KIND_TOPP) {
    const bool hist = md.kind == KIND_TOPP;
    double t = 0.0;
    int bl = NBIN, bh = -1;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      if (MLXF_IDX(e) < end) {
        const float zp = fz<DT>(v[e], md.Tr);
        const float w = wexp(zp, mps);
        t += static_cast<double>(w);
        if (hist) {
          const int b = static_cast<int>(f2key(zp) >> 21);
          bl = min(bl, b);
          bh = max(bh, b);
          const unsigned long long q = quant(w);
          if (q) atomicAdd(&r1.hist[b], q);
        }
      }
    }
    const double ws = wave_sum(t);
    if (hist) {
      bl = wave_min(bl);
      bh = wave_max(bh);
    }
    if (lane == 0) {
      sh.rd2[wid] = ws;
      sh.bmin[wid] = bl;
      sh.bmax[wid] = bh;
    }
  } else if (md.kind == KIND_KHIST) {
    int bl = CNT_BINS, bh = -1;
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
      if (MLXF_IDX(e) < end) {
        const int b = static_cast<int>(f2key(v[e]) >> 20);
        bl = min(bl, b);
        bh = max(bh, b);
        atomicAdd(&r1.cnt[b], 1u);
      }
    }
    bl = wave_min(bl);
    bh = wave_max(bh);
    if (lane == 0) {
      sh.bmin[wid] = bl;
      sh.bmax[wid] = bh;
    }
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
    // only the occupied bins are stored; the range goes with the slice record
    int bl = sh.bmin[0], bh = sh.bmax[0];
#pragma unroll
    for (int w2 = 1; w2 < WAVES; ++w2) {
      bl = min(bl, sh.bmin[w2]);
      bh = max(bh, sh.bmax[w2]);
    }
    const size_t off = (static_cast<size_t>(r) * S + s) * NBIN;
    for (int b = bl + tid; b <= bh; b += THREADS) st_dev(a.hist + off + b, r1.hist[b]);
    ncand = bh < bl ? 0xffffu : static_cast<unsigned int>(bl) | (static_cast<unsigned int>(bh) << 16);
  } else if (md.kind == KIND_KHIST) {
    // the occupied bins of the count histogram of z keys, as 32-bit counts
    int bl = sh.bmin[0], bh = sh.bmax[0];
#pragma unroll
    for (int w2 = 1; w2 < WAVES; ++w2) {
      bl = min(bl, sh.bmin[w2]);
      bh = max(bh, sh.bmax[w2]);
    }
    unsigned int* hc = reinterpret_cast<unsigned int*>(a.hist + (static_cast<size_t>(r) * S + s) * NBIN);
    for (int b = bl + tid; b <= bh; b += THREADS)
      __hip_atomic_store(hc + b, r1.cnt[b], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    ncand = bh < bl ? 0xffffu : static_cast<unsigned int>(bl) | (static_cast<unsigned int>(bh) << 16);
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
  if (sh.ticket != static_cast<unsigned int>(S - 1)) return false;
  if (tid == 0) {
    __hip_atomic_store(a.ctr + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next call
    sh.args = a;
    sh.md = md;
  }
  __syncthreads();
  finish_row<DT, EPT, VECOK>(r, r0, r1, sh);
  return true;
}

// Second pass, one item = slice s of a queued row (top-p without top-k): the
// slice's mass above the bracket (its own histogram's bins above bhi, exact)
// and the bracket's elements, counted per z' value (value mode) or written out
// as candidates.  The row's last item resolves the row.
template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ void second_pass(const Args& a, int r, int s, Region0& r0, Region1& r1, Small& sh) {
  const int tid = threadIdx.x, lane = tid & 63;
  const int S = a.S;
  const Mode md = decode<DT>(a, r);
  const void* row = row_ptr<DT>(a, r);
  const unsigned long long* pl = a.plan + static_cast<size_t>(r) * PLAN_WORDS;
  const unsigned long long wk = ld_dev(pl + PL_KEYS), wmode = ld_dev(pl + PL_MODE);
  const unsigned int klo = static_cast<unsigned int>(wk), khi = static_cast<unsigned int>(wk >> 32);
  const bool has_hi = (wmode & 1ull) != 0;
  const bool khist = ((wmode >> 12) & 1ull) != 0;
  const int bhi = static_cast<int>((wmode >> 1) & 0x7ffull);
  const int nv = static_cast<int>((wmode >> 32) & 0x7ffull);
  const unsigned int vbase = static_cast<unsigned int>(wmode >> 43);
  const unsigned long long w1 =
      ld_dev(reinterpret_cast<const unsigned long long*>(a.rec + (r * S + s)) + 1);
  const unsigned int rg = static_cast<unsigned int>(w1 >> 32);
  const int rlo = static_cast<int>(rg & 0xffffu), rhi = static_cast<int>(rg >> 16);
  // mass above the bracket (top-p rows): this slice's histogram bins above bhi
  unsigned long long ab = 0;
  const unsigned long long* hs = a.hist + (static_cast<size_t>(r) * S + s) * NBIN;
  if (!khist)
    for (int b = max(bhi + 1, rlo) + tid; b <= rhi; b += THREADS) ab += ld_dev(hs + b);
  if (nv > 0)
    for (int v = tid; v < nv; v += THREADS) r0.vcnt[v] = 0u;
  if (tid == 0) sh.ncand = 0u;
  ab = block_sum<unsigned long long>(ab, sh.ru);  // (its barriers also publish the clears)
  // the bracket's elements
  const int beg = s * a.L, end = min(a.V, beg + a.L);
  constexpr int NIT = EPT / VEC;
  uint2* dst = a.cand + (static_cast<size_t>(r) * S + s) * a.L;
#pragma unroll
  for (int it = 0; it < NIT; ++it) {
    float z[VEC];
    const int i0 = beg + it * CHUNK + tid * VEC;
    load8<DT, VECOK>(row, i0, end, z);
#pragma unroll
    for (int j = 0; j < VEC; ++j) {
      const int i = i0 + j;
      const unsigned int zk = f2key(z[j]);
      const bool inr = i < end && zk >= klo && (!has_hi || zk < khi);
      unsigned int zpk = 0;
      if (inr) zpk = f2key(fz<DT>(z[j], md.Tr));
      if (nv > 0) {
        if (inr) atomicAdd(&r0.vcnt[(zpk >> vshift<DT>()) - vbase], 1u);
      } else {
        const unsigned long long bal = __ballot(inr);
        if (bal) {
          unsigned int basepos = 0;
          if (lane == 0) basepos = atomicAdd(&sh.ncand, static_cast<unsigned int>(__popcll(bal)));
          basepos = rdl(basepos, 0);
          if (inr) {
            const unsigned int pos =
                basepos + __builtin_amdgcn_mbcnt_hi(static_cast<unsigned int>(bal >> 32),
                                                    __builtin_amdgcn_mbcnt_lo(static_cast<unsigned int>(bal), 0u));
            st_dev(dst + pos, make_uint2(zpk, static_cast<unsigned int>(i)));
          }
        }
      }
    }
  }
  __syncthreads();
  if (nv > 0) {
    for (int w = tid; w < nv / 2; w += THREADS)
      st_dev(reinterpret_cast<unsigned long long*>(dst) + w, pack2(r0.vcnt[2 * w], r0.vcnt[2 * w + 1]));
  } else if (tid == 0) {
    __hip_atomic_store(a.ncand2 + (r * S + s), sh.ncand, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (tid == 0)
    st_dev(a.above + (r * S + s),
           static_cast<unsigned long long>(__double_as_longlong(static_cast<double>(ab) * QUNIT)));
  // ticket: the row's last item resolves the row
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0)
    sh.ticket = __hip_atomic_fetch_add(a.done2 + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (sh.ticket != static_cast<unsigned int>(S - 1)) return;
  if (tid == 0) {
    __hip_atomic_store(a.done2 + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // next call
    sh.args = a;
    sh.md = md;
  }
  if (tid < PLAN_WORDS) sh.plan[tid] = ld_dev(pl + tid);
  __syncthreads();
  resolve_row<DT, EPT, VECOK>(r, r0, r1, sh);
}

// Helpers: take second-pass items of any queued row, polling until every row is
// finished or the idle bound runs out.  No row depends on helpers (see
// drain_own); the workgroup that completes a row's last item resolves it.
// Take the items of one row until none is left.  A row's last slice does this
// for its own row after queueing it, so every item is taken by a running
// workgroup whatever the helpers do.
template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ void drain_own(const Args& a, int own_row, Region0& r0, Region1& r1, Small& sh) {
  const int tid = threadIdx.x;
  for (;;) {
    __syncthreads();
    if (tid == 0)
      sh.qitem = static_cast<int>(stamped_take(a.next2 + own_row, a.epoch, static_cast<unsigned int>(a.S)));
    __syncthreads();
    const int qi = sh.qitem;
    if (qi >= a.S) break;
    second_pass<DT, EPT, VECOK>(a, own_row, qi, r0, r1, sh);
  }
}

template <int DT, int EPT, bool VECOK>
__device__ __forceinline__ void drain(const Args& a, Region0& r0, Region1& r1, Small& sh) {
  constexpr bool wait = true;
  const int tid = threadIdx.x;
  const int S = a.S;
  unsigned int cursor = 0;
  int polls = 0;
  for (;;) {
    __syncthreads();
    if (tid == 0) {
      sh.rdone = stamped_get(a.gl + GL_ROWS, a.epoch);
      sh.qn = stamped_get(a.gl + GL_QRES, a.epoch);
      sh.qrow = static_cast<int>(stamped_get(a.gl + GL_HEAD, a.epoch));
    }
    __syncthreads();
    const unsigned int qn = sh.qn, rdone = sh.rdone;
    cursor = max(cursor, static_cast<unsigned int>(sh.qrow));
    bool worked = false;
    while (cursor < qn) {
      __syncthreads();
      if (tid == 0) {
        // a reserved slot is written right after its reservation
        unsigned int e = stamped_get(a.queue + cursor, a.epoch);
        for (int spin = 0; e == 0u && spin < (1 << 20); ++spin) {
          __builtin_amdgcn_s_sleep(2);
          e = stamped_get(a.queue + cursor, a.epoch);
        }
        int item = S;
        if (e != 0u) item = static_cast<int>(stamped_take(a.next2 + (e - 1u), a.epoch, static_cast<unsigned int>(S)));
        sh.qrow = static_cast<int>(e) - 1;
        sh.qitem = item;
      }
      __syncthreads();
      const int qr = sh.qrow, qi = sh.qitem;
      if (qr < 0 || qi >= S) {
        // the row has no items left: move the shared head past it if it points here
        if (tid == 0) {
          unsigned long long w = (static_cast<unsigned long long>(a.epoch) << 32) | cursor;
          __hip_atomic_compare_exchange_strong(a.gl + GL_HEAD, &w, w + 1ull, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
          if (cursor == 0u) {  // a head never stamped in this call reads as 0
            unsigned long long z = ld_dev(a.gl + GL_HEAD);
            if (static_cast<unsigned int>(z >> 32) != a.epoch)
              __hip_atomic_compare_exchange_strong(a.gl + GL_HEAD, &z, w + 1ull, __ATOMIC_RELAXED,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
        }
        ++cursor;
        continue;
      }
      second_pass<DT, EPT, VECOK>(a, qr, qi, r0, r1, sh);
      worked = true;
    }
    if (!wait || rdone >= static_cast<unsigned int>(a.B)) break;
    if (worked) {
      polls = 0;
    } else {
      if (++polls > IDLE_LIMIT) break;
      // back off: idle helpers poll the shared counters less often
      if (polls < 8)
        __builtin_amdgcn_s_sleep(8);
      else
        __builtin_amdgcn_s_sleep(64);
    }
  }
}

// One launch: the first B*S workgroups run the first pass (row-major); those
// that finish a row with a second pass then take that row's items.  The remaining
// workgroups are helpers that only take second-pass items, and leave at once
// unless some row of this call flagged a second pass.
template <int DT, int EPT, bool VECOK>
__global__ __launch_bounds__(THREADS, 2) void k_sample(Args a) {
  __shared__ Region0 r0;
  __shared__ Region1 r1;
  __shared__ Small sh;
  const int bid = static_cast<int>(blockIdx.x);
  const int n1 = a.B * a.S;
  if (bid < n1) {
    const int r = bid / a.S;
    if (first_pass<DT, EPT, VECOK>(a, r, bid - r * a.S, r0, r1, sh)) {
      const int kind = sh.md.kind;
      if (kind == KIND_TOPP && sh.md.pr > 0.0f)
        drain_own<DT, EPT, VECOK>(a, r, r0, r1, sh);
      else if (kind == KIND_KHIST)
        drain_own<DT, EPT, VECOK>(a, r, r0, r1, sh);
    }
  } else {
    if (threadIdx.x == 0) sh.qn = stamped_get(a.gl + GL_NEED, a.epoch);
    __syncthreads();
    if (sh.qn != 0u) drain<DT, EPT, VECOK>(a, r0, r1, sh);
  }
}

// Zero the per-row counters of a fresh workspace.
__global__ void k_zero(unsigned int* p, size_t n) {
  const size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// ================================================================ host side ==

struct Layout {
  int S, L, EPT;
  size_t off_ctr, off_done2, off_next2, off_gl, off_queue, off_rec, off_list, off_hist, off_cand,
      off_plan, off_above, off_ncand2, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// the zero-initialised head of the workspace: per-row tickets (two arrays of
// 65536 32-bit counters), item counters and queue slots (65536 64-bit words
// each) and the call-wide counters
constexpr size_t ROWS_MAX = 65536;
constexpr size_t CTR_BYTES_MAX =
    2 * ROWS_MAX * sizeof(unsigned int) + 2 * ROWS_MAX * sizeof(unsigned long long) +
    GL_WORDS * sizeof(unsigned long long);

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
  // First, at offsets that do not depend on the shape: the three per-row
  // counter arrays, which must read zero before every call (the workspace is
  // zeroed once; every call leaves them at zero).  Fixed offsets keep that true
  // when one workspace serves calls of different shapes.
  const size_t nb = B > 0 ? static_cast<size_t>(B) : 1;
  l.off_ctr = 0;
  l.off_done2 = ROWS_MAX * sizeof(unsigned int);
  l.off_next2 = 2 * ROWS_MAX * sizeof(unsigned int);
  l.off_queue = l.off_next2 + ROWS_MAX * sizeof(unsigned long long);
  l.off_gl = l.off_queue + ROWS_MAX * sizeof(unsigned long long);
  o = align256(CTR_BYTES_MAX);
  l.off_rec = o;
  o = align256(o + sizeof(SliceRec) * BS);
  l.off_list = o;
  o = align256(o + sizeof(unsigned long long) * BS * LIST);
  l.off_hist = o;
  o = align256(o + sizeof(unsigned long long) * BS * NBIN);
  l.off_cand = o;
  o = align256(o + sizeof(uint2) * BS * l.L);
  l.off_plan = o;
  o = align256(o + sizeof(unsigned long long) * PLAN_WORDS * nb);
  l.off_above = o;
  o = align256(o + sizeof(double) * BS);
  l.off_ncand2 = o;
  o = align256(o + sizeof(unsigned int) * BS);
  l.total = o;
  return l;
}

// A fresh stamp per call (never 0, which a zeroed workspace holds).
unsigned int next_epoch() {
  static std::atomic<unsigned int> counter{0};
  unsigned int e;
  do {
    e = counter.fetch_add(1u, std::memory_order_relaxed) + 1u;
  } while (e == 0u);
  return e;
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

// Helper workgroups (at most 256) are added when some row can have a second
// pass (top-p without top-k, or top-k with k > 63).
template <int DT, int EPT>
hipError_t launch_ept(Args a, bool vecok, hipStream_t st) {
  const int n1 = a.B * a.S;
  a.helpers = (a.T != nullptr && (a.p != nullptr || a.k != nullptr)) ? (n1 < 256 ? n1 : 256) : 0;
  const dim3 grid(n1 + a.helpers);
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
    a.done2 = reinterpret_cast<unsigned int*>(ws + l.off_done2);
    a.next2 = reinterpret_cast<unsigned long long*>(ws + l.off_next2);
    a.queue = reinterpret_cast<unsigned long long*>(ws + l.off_queue);
    a.gl = reinterpret_cast<unsigned long long*>(ws + l.off_gl);
    a.epoch = next_epoch();
    a.plan = reinterpret_cast<unsigned long long*>(ws + l.off_plan);
    a.above = reinterpret_cast<double*>(ws + l.off_above);
    a.ncand2 = reinterpret_cast<unsigned int*>(ws + l.off_ncand2);
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
