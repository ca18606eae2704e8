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
// Each row is split over G workgroups of 1024 threads and the work runs as a
// sequence of launches, one per phase (see the filter section below): the
// top-k threshold and the nucleus cutoff are radix selections over 32-bit
// order keys (11-bit digits; two levels decide a 16-bit dtype's key, three an
// fp32 one), each level a histogram of counts or of fixed-point masses built
// per slice in LDS and summed over the slices through the workspace, and the
// last phase writes z' or -inf.  Two things keep the passes near the rate the
// memory allows:
//  - the radix histograms hold RC copies of each bin, lane l adding into copy
//    l % RC: a row's first digits fall into a few bins, and lanes adding into
//    one LDS word are served one after another;
//  - every pass reads 8-element units with 16-byte loads; where index order
//    matters (a partial tie group) wave w takes the contiguous segment
//    [w S, (w + 1) S) of its slice and ranks its tied elements by a wave
//    prefix sum, after the tie counts of the segments before it (counted by
//    the phase before).
#include <hip/hip_runtime.h>

#include <cstdlib>
#include <cstring>
#include <string>

#include "sampler_impl.hpp"

namespace mlxf {
namespace {

constexpr int FT = 1024;      // threads per workgroup
constexpr int FW = FT / 64;   // waves
constexpr int NBIN = 2048;    // bins of a radix level (11-bit digits)
constexpr int RC = 4;         // copies of each radix bin (lane l adds into copy l % RC)
constexpr int FU8 = 1;        // 8-element units per lane per loop step (2 and 4 measured slower)

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
  bool vec;   // 16-byte loads: the logits' base and row stride allow them
  bool ovec;  // 16-byte stores: the output's base and row stride allow them
};

struct FLds {
  unsigned int hc[NBIN * RC];        // bin d, copy c at d * RC + c
  unsigned long long hm[NBIN * RC];
  unsigned long long u64r[FW];
  float fr[FW];
  unsigned int sel[2];          // the chosen digit and its count
  unsigned long long sel64[1];  // the measure above it
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
// n (<= 8) consecutive values from i0 (i0 % 8 == 0), each representable in
// the dtype: whole units in 16-byte stores where the row allows them.
template <int DT>
__device__ __forceinline__ void st8(void* row, bool vec, int i0, const float* v, int n) {
  if (vec && n == 8) {
    uint4* p = reinterpret_cast<uint4*>(static_cast<char*>(row) + static_cast<size_t>(i0) * elem_size<DT>());
    if constexpr (DT == MLXF_DTYPE_F32) {
      p[0] = make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
      p[1] = make_uint4(__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7]));
    } else {
      unsigned int h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if constexpr (DT == MLXF_DTYPE_BF16)
          h[e] = __float_as_uint(v[e]) >> 16;
        else
          h[e] = static_cast<unsigned int>(__half_as_ushort(__float2half_rn(v[e])));
      }
      p[0] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e)
      if (e < n) st1<DT>(row, i0 + e, v[e]);
  }
}

// Order key of a stored z': -0 and +0 compare equal (as the reference's float
// comparisons do), so they share a key.
__device__ __forceinline__ unsigned int okey(float zp) { return f2key(zp + 0.0f); }

// A row as the passes read it: 8-element units of raw storage (two 16-byte
// loads for fp32, one for the 16-bit types, where the row's base and stride
// allow; element loads otherwise), each decoded value passed through xf.
template <int DT, typename Xf>
struct RowSrc {
  const void* row;
  bool vec;
  Xf xf;
  __device__ __forceinline__ void load(int i0, int end, Raw8<DT>& r) const {
    if (vec)
      load_raw<DT, true>(row, i0, end, r);
    else
      load_raw<DT, false>(row, i0, end, r);
  }
  __device__ __forceinline__ float at(int i) const {
    Raw8<DT> r;
    load_raw<DT, false>(row, i, i + 1, r);
    float v[8];
    decode8_nan<DT>(r, v);
    return xf(v[0]);
  }
};
template <int DT, typename Xf>
__device__ __forceinline__ RowSrc<DT, Xf> row_src(const void* row, bool vec, Xf xf) {
  return RowSrc<DT, Xf>{row, vec, xf};
}

// fn(i, value) for every i in [lo, hi) (lo % 8 == 0), lane t taking the units
// t, t + FT, ...; FU8 units per lane per step are loaded before the first is
// used (one 16- or 32-byte unit measured fastest: the 16 waves of a CU keep
// enough loads in flight).
template <int DT, typename Xf, typename Fn>
__device__ __forceinline__ void row_pass(int lo, int hi, const RowSrc<DT, Xf>& src, Fn fn) {
  const int nu = (hi - lo + 7) >> 3;
  for (int j0 = static_cast<int>(threadIdx.x); j0 < nu; j0 += FU8 * FT) {
    Raw8<DT> raw[FU8];
#pragma unroll
    for (int q = 0; q < FU8; ++q) {
      const int j = j0 + q * FT;
      if (j < nu) src.load(lo + 8 * j, hi, raw[q]);
    }
#pragma unroll
    for (int q = 0; q < FU8; ++q) {
      const int j = j0 + q * FT;
      if (j < nu) {
        float v[8];
        decode8_nan<DT>(raw[q], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = lo + 8 * j + e;
          if (i < hi) fn(i, src.xf(v[e]));
        }
      }
    }
  }
}

// Over wave w's contiguous segment [s0, s1) (s0 % 8 == 0) in index order,
// 512 elements per step, 8 consecutive ones per lane: fn(i0, v, n) with the
// lane's first index, its 8 values and how many of them are in the segment
// (0 to 8).  Every lane of the wave takes part in every step, so fn may use
// wave operations.
template <int DT, typename Xf, typename Fn>
__device__ __forceinline__ void seg_pass(int s0, int s1, const RowSrc<DT, Xf>& src, Fn fn) {
  const int lane = static_cast<int>(threadIdx.x) & 63;
  for (int b = s0; b < s1; b += FU8 * 512) {
    Raw8<DT> raw[FU8];
#pragma unroll
    for (int q = 0; q < FU8; ++q) {
      const int i0 = b + q * 512 + 8 * lane;
      if (i0 < s1) src.load(i0, s1, raw[q]);
    }
#pragma unroll
    for (int q = 0; q < FU8; ++q) {
      const int i0 = b + q * 512 + 8 * lane;
      float v[8];
      if (i0 < s1) {
        decode8_nan<DT>(raw[q], v);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = src.xf(v[e]);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = -INFINITY;
      }
      fn(i0, v, min(max(s1 - i0, 0), 8));
    }
  }
}

template <typename T>
__device__ __forceinline__ T fsum(T x, T* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  x = wave_sum(x);
  __syncthreads();
  if (lane == 0) red[wid] = x;
  __syncthreads();
  return rdl(row_sum16(lane < FW ? red[lane & (FW - 1)] : T(0)), 0);
}

// Wave w's contiguous segment [*s0, *s1) of the range [lo, hi) (lo % 8 == 0),
// in whole 512-element steps.
__device__ __forceinline__ void wave_segment(int lo, int hi, int* s0, int* s1) {
  const int S = ((hi - lo + FW * 512 - 1) / (FW * 512)) * 512;
  *s0 = min(lo + (static_cast<int>(threadIdx.x) >> 6) * S, hi);
  *s1 = min(*s0 + S, hi);
}

// Index-order ranks inside one seg_pass step: each lane's count c of marked
// elements among its 8; returns the marked elements of the lower lanes, and
// the step's total in *tot.
__device__ __forceinline__ unsigned int lanes_before(unsigned int c, unsigned int* tot) {
  const int inc = wave_incl_scan_dpp(static_cast<int>(c));
  *tot = static_cast<unsigned int>(rdl(inc, 63));
  return static_cast<unsigned int>(inc) - c;
}

// Each wave's count of the elements of its segment whose value satisfies
// pred, stored at cnt[g FW + w] for the next phases.
template <int DT, typename Xf, typename Pred>
__device__ void seg_counts(int lo, int hi, int g, const RowSrc<DT, Xf>& src, Pred pred, unsigned int* cnt) {
  int s0, s1;
  wave_segment(lo, hi, &s0, &s1);
  unsigned int mine = 0u;
  seg_pass(s0, s1, src, [&](int, const float* v, int n) {
#pragma unroll
    for (int e = 0; e < 8; ++e) mine += (e < n && pred(v[e])) ? 1u : 0u;
  });
  mine = wave_sum(mine);
  if ((threadIdx.x & 63) == 0) cnt[g * FW + (threadIdx.x >> 6)] = mine;
}

// The sum of cnt[0 .. g FW + w): the counted elements of the wave segments
// before this wave's, in index order (whole wave).
__device__ __forceinline__ unsigned int segs_before(const unsigned int* cnt, int g) {
  const int idx = g * FW + (static_cast<int>(threadIdx.x) >> 6), lane = threadIdx.x & 63;
  unsigned int t = 0u;
  for (int q = lane; q < idx; q += 64) t += cnt[q];
  return wave_sum(t);
}

// ---- the filter calls: G workgroups per row, one kernel per phase.
// Workgroup g of row r takes the slice [g L, (g + 1) L) of the row.  Every
// phase recomputes z' from the input (the division is deterministic), so the
// output is written only by the last phase and may be the input itself.  A
// radix level's histogram is built per slice in LDS and written out whole
// (every bin, zeros included); the next phase sums the G slice histograms of
// its row (integer sums, so the order does not matter), picks the digit, and
// builds the next level.  Workgroup 0 of a row stores the selection's state
// after each level for the phases after it; states and histograms alternate
// between two slots, so no phase reads a slot it writes.

constexpr int FG_MAX = 16;   // workgroups per row at most

// A radix selection's state after a level: the digits chosen so far (prefix
// under mask), the target left below them, the measure above them, the count
// of candidates with the chosen key (after the last level), the target.
struct FSel {
  unsigned int prefix, mask, cnt, pad;
  unsigned long long rem, abv, tgt;
};

struct FRow {
  FSel sk[2], sp[2];          // top-k and top-p states after level j at [j & 1]
  float mxp[FG_MAX];          // slice maxima of z'
  unsigned int tiec[FG_MAX * FW];  // per wave segment (slice g, wave w at g FW + w): counts of a cutoff's key
};

enum FPhase { FP_MAX, FP_K1, FP_K2, FP_K3, FP_P0, FP_P1, FP_P2, FP_P3, FP_TIES, FP_FIN };

// Radix levels a dtype needs: the order key of a 16-bit value has its low
// bits fixed (bf16: 16, f16: 13; zeros for a non-negative value, ones for a
// negative one), so the two 11-bit digits decide it; fp32 takes all three
// levels.  complete_key fills the bits below the decided digits.
__host__ __device__ constexpr int nlev(int dt) { return dt == MLXF_DTYPE_F32 ? 3 : 2; }
template <int DT>
__device__ __forceinline__ unsigned int complete_key(unsigned int prefix) {
  if constexpr (nlev(DT) == 3) return prefix;
  constexpr unsigned int low = 0x3ffu;  // below the second level's digit (bits 10-20)
  return (prefix & 0x80000000u) ? prefix : (prefix | low);
}

struct FWs {
  FRow* rows;               // [B]
  unsigned int* hc;         // [B][2][G][NBIN]
  unsigned long long* hm;   // [B][2][G][NBIN]
  int G;
};

__host__ __device__ inline size_t fws_align(size_t x) { return (x + 255) & ~static_cast<size_t>(255); }

// Workgroups per row: the B G workgroups fill the CUs (one per CU, as each
// holds its radix histograms in most of a CU's LDS) with slices of at least
// 4096 elements.
__host__ __device__ inline int filter_groups(int B, int V) {
  int G = B > 0 ? (256 + B - 1) / B : 1;
  const int gv = (V + 4095) / 4096;
  G = G < gv ? G : gv;
  return G < 1 ? 1 : (G > FG_MAX ? FG_MAX : G);
}

__host__ __device__ inline size_t filter_ws_bytes(int B, int V) {
  const size_t G = static_cast<size_t>(filter_groups(B, V));
  const size_t nb = static_cast<size_t>(B) * 2 * G * NBIN;
  return fws_align(static_cast<size_t>(B) * sizeof(FRow)) + fws_align(nb * 4) + fws_align(nb * 8);
}

// The radix levels over the 32-bit order key: 11-bit digits at bits 21-31
// and 10-20, then a 10-bit one at bits 0-9.
__host__ __device__ constexpr int lvl_shift(int l) { return l == 1 ? 21 : (l == 2 ? 10 : 0); }
__host__ __device__ constexpr unsigned int lvl_mask(int l) { return l < 3 ? 0x7ffu : 0x3ffu; }

// Sum the G slice histograms of level l for this row and choose its digit:
// the state s moves to the digit d whose measure (count, or mass when MASS)
// brings the measure above it from below s.rem to at least s.rem.  With
// FROM_TOTAL the target is first set from the candidates' whole measure W:
// max(1, ceil(p W)) (the nucleus's first level).  Thread t takes the digits
// 2047 - 2t and 2046 - 2t (descending order).
template <bool MASS, bool FROM_TOTAL>
__device__ FSel select_level(FSel s, int l, const unsigned int* hc, const unsigned long long* hm, int G, float pr,
                             FLds& sh) {
  const int tid = threadIdx.x;
  const unsigned int d1 = static_cast<unsigned int>(NBIN - 1 - 2 * tid), d0 = d1 - 1u;
  unsigned int c1 = 0u, c0 = 0u;
  unsigned long long m1 = 0ull, m0 = 0ull;
  for (int g = 0; g < G; ++g) {
    c1 += hc[g * NBIN + d1];
    c0 += hc[g * NBIN + d0];
    if (MASS) {
      m1 += hm[g * NBIN + d1];
      m0 += hm[g * NBIN + d0];
    }
  }
  if (!MASS) {
    m1 = c1;
    m0 = c0;
  }
  __syncthreads();  // sh.sel may still be read by the caller's last use
  if (tid == 0) {
    sh.sel[0] = 0u;
    sh.sel[1] = 0u;
    sh.sel64[0] = 0ull;
  }
  unsigned long long tot;
  const unsigned long long excl = rh::bscan(m1 + m0, sh.u64r, &tot);  // (barriers inside)
  if (FROM_TOTAL) {
    unsigned long long PW = static_cast<unsigned long long>(ceil(static_cast<double>(pr) * static_cast<double>(tot)));
    if (PW < 1ull) PW = 1ull;
    s.rem = PW;
    s.tgt = PW;
  }
  if (excl < s.rem && s.rem <= excl + m1) {
    sh.sel[0] = d1;
    sh.sel64[0] = excl;
    sh.sel[1] = c1;
  } else if (excl + m1 < s.rem && s.rem <= excl + m1 + m0) {
    sh.sel[0] = d0;
    sh.sel64[0] = excl + m1;
    sh.sel[1] = c0;
  }
  __syncthreads();
  const unsigned int dd = sh.sel[0];
  const unsigned long long ex = sh.sel64[0];
  s.cnt = sh.sel[1];
  s.rem -= ex;
  s.abv += ex;
  s.prefix |= dd << lvl_shift(l);
  s.mask |= lvl_mask(l) << lvl_shift(l);
  return s;
}

// This slice's level-l histogram of the candidates (key under s's prefix,
// in(zp, key)) into hc / hm (this workgroup's NBIN bins); extra(zp) sees every
// element of the slice on the way.
struct NoExtra {
  __device__ void operator()(float) const {}
};

template <bool MASS, typename Load, typename In, typename Mass, typename Extra = NoExtra>
__device__ void slice_hist(int lo, int hi, int l, FSel s, Load load, In in, Mass massf, unsigned int* hc,
                           unsigned long long* hm, FLds& sh, Extra extra = Extra{}) {
  const int tid = threadIdx.x;
  const unsigned int cpy = static_cast<unsigned int>(tid) & (RC - 1);
  __syncthreads();
  for (int j = tid; j < NBIN * RC; j += FT) {
    sh.hc[j] = 0u;
    if (MASS) sh.hm[j] = 0ull;
  }
  __syncthreads();
  const unsigned int prefix = s.prefix, mask = s.mask;
  const int shift = lvl_shift(l);
  const unsigned int dmask = lvl_mask(l);
  row_pass(lo, hi, load, [&](int, float zp) {
    extra(zp);
    const unsigned int key = okey(zp);
    if ((key & mask) == prefix && in(zp, key)) {
      const unsigned int d = ((key >> shift) & dmask) * RC + cpy;
      __hip_atomic_fetch_add(&sh.hc[d], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if (MASS) {
        const unsigned long long m = massf(zp);
        if (m) __hip_atomic_fetch_add(&sh.hm[d], m, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
    }
  });
  __syncthreads();
  for (int d = tid; d < NBIN; d += FT) {
    unsigned int c = 0u;
    unsigned long long m = 0ull;
#pragma unroll
    for (int k = 0; k < RC; ++k) {
      c += sh.hc[d * RC + k];
      if (MASS) m += sh.hm[d * RC + k];
    }
    hc[d] = c;
    if (MASS) hm[d] = m;
  }
}

template <int DT>
__global__ __launch_bounds__(FT, 1) void k_filter(FArgs f, FWs ws, int ph) {
  __shared__ FLds sh;
  const int tid = threadIdx.x;
  const int r = static_cast<int>(blockIdx.x), g = static_cast<int>(blockIdx.y);
  const int V = f.V, G = ws.G;
  const int L = (((V + G - 1) / G) + 63) & ~63;
  const int lo = min(g * L, V), hi = min(lo + L, V);
  const void* irow = static_cast<const char*>(f.logits) + static_cast<size_t>(r) * f.row_stride * elem_size<DT>();
  void* orow = static_cast<char*>(f.out) + static_cast<size_t>(r) * f.out_stride * elem_size<DT>();
  FRow& row = ws.rows[r];
  unsigned int* hc0 = ws.hc + static_cast<size_t>(r) * 2 * G * NBIN;
  unsigned long long* hm0 = ws.hm + static_cast<size_t>(r) * 2 * G * NBIN;
  auto hcs = [&](int slot) { return hc0 + static_cast<size_t>(slot) * G * NBIN; };
  auto hms = [&](int slot) { return hm0 + static_cast<size_t>(slot) * G * NBIN; };

  // ---- the row's parameters (the sampling call's sentinels)
  const float T = f.T ? f.T[r] : f.Ts;
  const float Tr = round_dt<DT>(T);
  const bool div = __builtin_isfinite(T) && T > 0.0f && Tr > 0.0f;
  const int k0 = f.k ? f.k[r] : f.ks;
  const int kk = k0 > 0 ? (k0 < V ? k0 : V) : 0;
  const bool tk_on = kk > 0 && kk < V;
  // (a p that rounds to 1 in the dtype keeps every element: every prior mass
  // is below the whole mass.  With integer masses the elements of zero mass
  // would reach it, so the filter is off then.)
  const float p = f.p ? f.p[r] : f.ps;
  const float pr = round_dt<DT>(p);
  const bool topp = p > 0.0f && p < 1.0f && pr < 1.0f;
  const float mp = f.minp ? f.minp[r] : f.mps;
  const float mr = (mp > 0.0f && mp <= 1.0f) ? round_dt<DT>(mp) : 0.0f;
  // z' (NaN read as -inf)
  const auto src = row_src<DT>(irow, f.vec, [=](float z) {
    z = z != z ? -INFINITY : z;
    return div ? round_dt<DT>(z / Tr) : z;
  });
  auto all = [](float, unsigned int) { return true; };
  auto nomass = [](float) { return 0ull; };

  if (ph == FP_MAX) {
    // ---- the slice's max of z', and the top-k's first level
    float mx = -INFINITY;
    row_pass(lo, hi, src, [&](int, float zp) { mx = fmaxf(mx, zp); });
    const float w = wave_max(mx);
    if ((tid & 63) == 0) sh.fr[tid >> 6] = w;
    __syncthreads();
    const float m = rdl(row_max16(sh.fr[tid & (FW - 1)]), 0);
    if (tid == 0) row.mxp[g] = m;
    if (tk_on) {
      FSel s{};
      slice_hist<false>(lo, hi, 1, s, src, all, nomass, hcs(0) + g * NBIN, nullptr, sh);
    }
    return;
  }
  constexpr int NL = nlev(DT);
  if (ph >= FP_K1 && ph <= FP_K3) {
    // ---- top-k level l = ph (l < NL): choose digit l from slot (l - 1) & 1,
    // build level l + 1 into slot l & 1 (src/sample/sampler.cpp:63-68)
    if (!tk_on) return;
    const int l = ph - FP_K1 + 1;
    FSel s{};
    s.rem = s.tgt = static_cast<unsigned long long>(kk);
    if (l > 1) s = row.sk[(l - 1) & 1];
    s = select_level<false, false>(s, l, hcs((l - 1) & 1), nullptr, G, 0.0f, sh);
    if (g == 0 && tid == 0) row.sk[l & 1] = s;
    slice_hist<false>(lo, hi, l + 1, s, src, all, nomass, hcs(l & 1) + g * NBIN, nullptr, sh);
    return;
  }

  // ---- the row max (every phase from here sums the slices the same way)
  float Mp = -INFINITY;
  for (int q = 0; q < G; ++q) Mp = fmaxf(Mp, row.mxp[q]);
  const bool minf = Mp == INFINITY;
  const float nc = minf ? 0.0f : -(Mp * LOG2E);
  auto massf = [&](float zp) -> unsigned long long { return q40(wfun(zp + 0.0f, Mp, nc, minf)); };
  const bool live = Mp != -INFINITY;  // a row of -inf (or NaN) keeps everything
  const bool tp_on = topp && live;

  if (ph == FP_P0) {
    // ---- top-k's last digit, then the nucleus's first level over the top-k
    // survivors (src/sample/sampler.cpp:70-85)
    unsigned int tk = 0u;
    if (tk_on) {
      FSel s = select_level<false, false>(row.sk[(NL - 1) & 1], NL, hcs((NL - 1) & 1), nullptr, G, 0.0f,
                                          sh);
      s.prefix = complete_key<DT>(s.prefix);
      if (g == 0 && tid == 0) row.sk[NL & 1] = s;
      tk = s.prefix;
    }
    if (tp_on) {
      FSel s{};
      slice_hist<true>(lo, hi, 1, s, src, [tk](float, unsigned int key) { return key >= tk; }, massf,
                       hcs(NL & 1) + g * NBIN, hms(NL & 1) + g * NBIN, sh);
    }
    return;
  }
  const unsigned int tk = tk_on ? row.sk[NL & 1].prefix : 0u;
  auto above_tk = [tk](float, unsigned int key) { return key >= tk; };
  if (ph >= FP_P1 && ph <= FP_P3) {
    // ---- nucleus level l: keep while the mass before an element, in (z'
    // desc, index asc) order, is below ceil(p W)
    if (!tp_on) return;
    const int l = ph - FP_P1 + 1;
    FSel s;
    if (l == 1) {
      s = FSel{};
      s = select_level<true, true>(s, 1, hcs(NL & 1), hms(NL & 1), G, pr, sh);
    } else {
      const int in = (NL + l - 1) & 1;
      s = select_level<true, false>(row.sp[(l - 1) & 1], l, hcs(in), hms(in), G, pr, sh);
    }
    if (g == 0 && tid == 0) row.sp[l & 1] = s;
    const int outs = (NL + l) & 1;
    slice_hist<true>(lo, hi, l + 1, s, src, above_tk, massf, hcs(outs) + g * NBIN, hms(outs) + g * NBIN,
                     sh);
    return;
  }

  // the nucleus cutoff: keys above ck kept, key ck keeps its first tkeep in
  // index order (all of them: tkeep = ~0)
  auto cutoff = [&](const FSel& s, unsigned int* ck, unsigned int* tkeep) {
    *ck = s.prefix;
    const unsigned long long wt = massf(key2f(s.prefix));
    const unsigned int t = ties_kept(s.tgt > s.abv ? s.tgt - s.abv : 0ull, wt, s.cnt);
    *tkeep = t >= s.cnt ? 0xffffffffu : t;
  };
  if (ph == FP_TIES) {
    // ---- the nucleus's last digit, and each wave segment's count of the
    // cutoff key when the cutoff's tie group is kept in part
    if (!tp_on) return;
    FSel s = select_level<true, false>(row.sp[(NL - 1) & 1], NL, hcs((2 * NL - 1) & 1),
                                       hms((2 * NL - 1) & 1), G, pr, sh);
    s.prefix = complete_key<DT>(s.prefix);
    if (g == 0 && tid == 0) row.sp[NL & 1] = s;
    unsigned int ck, tkeep;
    cutoff(s, &ck, &tkeep);
    if (tkeep == 0xffffffffu) return;
    seg_counts(lo, hi, g, src, [&](float zp) { return okey(zp) == ck; }, row.tiec);
    return;
  }

  // ---- FP_FIN: z', or -inf over every removed entry.  The partial tie
  // group keeps its first tkeep in index order: a tied element's rank is the
  // ties of the wave segments before its own (lower slices, then lower waves;
  // counted by FP_TIES), and those before it in its own segment
  unsigned int ck = 0u, tkeep = 0xffffffffu;
  if (tp_on) cutoff(row.sp[NL & 1], &ck, &tkeep);
  const bool filt = live && (tk_on || tp_on || mr > 0.0f);
  // min_p after them (src/sample/sampler.cpp:87-93): the weights that reach
  // min_p times the max's own weight
  const float thr = filt && mr > 0.0f ? minp_thr(mr, Mp, nc, minf) : 0.0f;
  const bool partial = tkeep != 0xffffffffu;
  int s0, s1;
  wave_segment(lo, hi, &s0, &s1);
  unsigned int rank = 0u;
  if (partial) rank = segs_before(row.tiec, g);
  seg_pass(s0, s1, src, [&](int i0, const float* v, int n) {
    bool keep[8];
    unsigned int c = 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      keep[e] = true;
      if (filt) {
        const unsigned int key = okey(v[e]);
        keep[e] = key >= tk && (!tp_on || key >= ck);
        if (mr > 0.0f) keep[e] = keep[e] && wfun(v[e] + 0.0f, Mp, nc, minf) >= thr;
        if (partial) c += (e < n && key == ck) ? 1u : 0u;
      }
    }
    if (partial) {
      // the tied elements in index order: the lower lanes' first, then this
      // lane's own
      unsigned int tot;
      unsigned int my = rank + lanes_before(c, &tot);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        if (e < n && okey(v[e]) == ck) {
          keep[e] = keep[e] && my < tkeep;
          ++my;
        }
      }
      rank += tot;
    }
    float w[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = keep[e] ? v[e] : -INFINITY;
    st8<DT>(orow, f.ovec, i0, w, n);
  });
}

// ---------------------------------------------------------------------------
// top_logprobs wider than the sampling kernels' best-64 lists (64 < K <= 4096):
// top_k_logprobs (src/sample/sampler.cpp:30-38; K = min(top_logprobs, V) at
// :52) as launches of their own after the sampling kernels, G workgroups per
// row as in the filter calls: the slice maxima of the unscaled row with the
// first radix level of the K-th largest logit; the slices' sums of exp(z - M)
// (fp32 exponentials, as the sampling kernels take them, summed in fp64) with
// the second level; the third level (fp32); the last digit
// with the slices' counts of the K-th logit's tie group; the gather of
// the K entries (every logit above the K-th, then the tied ones in index
// order) into the row's list in the workspace; and one workgroup per row that
// sorts the list by (logit desc, index asc) with a bitonic network in LDS and
// writes (id, logit - LSE), columns past the row's K as id -1 and -inf.

constexpr int TOPK_WIDE_MAX = 4096;
static_assert(TOPK_WIDE_MAX / 2 <= 2 * FT, "the sort gives each thread at most two pairs");

enum WPhase { W_MAX, W_K1, W_K2, W_K3, W_TIES, W_GATHER, W_SORT };

struct WRow {
  FRow f;
  double lsep[FG_MAX];        // slice sums of exp(z - M)
  unsigned int n, pad[63];    // entries gathered so far
};

struct WWs {
  WRow* rows;                 // [B]
  unsigned int* hc;           // [B][2][G][NBIN]
  unsigned long long* list;   // [B][K_max]: (key << 32) | ~index
  int G;
};

struct TkLds {
  FLds f;
  unsigned long long ent[TOPK_WIDE_MAX];  // (key << 32) | ~index: one unsigned order, larger first
  unsigned int n, base;
  double dr[FW];
};

__host__ __device__ inline size_t wide_ws_bytes(int B, int V, int K_max) {
  const size_t G = static_cast<size_t>(filter_groups(B, V));
  const size_t nb = static_cast<size_t>(B) * 2 * G * NBIN;
  return fws_align(static_cast<size_t>(B) * sizeof(WRow)) + fws_align(nb * 4) +
         fws_align(static_cast<size_t>(B) * K_max * 8);
}

template <int DT>
__global__ __launch_bounds__(FT, 1) void k_topk_wide(const void* logits, long long row_stride, int V, const int* tlp,
                                                     int K_max, int* top_ids, float* top_lp, WWs ws, int ph,
                                                     bool vec) {
  __shared__ TkLds sh;
  const int tid = threadIdx.x;
  const int r = static_cast<int>(blockIdx.x), g = static_cast<int>(blockIdx.y);
  const int G = ws.G;
  const int L = (((V + G - 1) / G) + 63) & ~63;
  const int lo = min(g * L, V), hi = min(lo + L, V);
  const void* row = static_cast<const char*>(logits) + static_cast<size_t>(r) * row_stride * elem_size<DT>();
  WRow& wr = ws.rows[r];
  FRow& fr = wr.f;
  unsigned int* hc0 = ws.hc + static_cast<size_t>(r) * 2 * G * NBIN;
  auto hcs = [&](int slot) { return hc0 + static_cast<size_t>(slot) * G * NBIN; };
  unsigned long long* lst = ws.list + static_cast<size_t>(r) * K_max;
  const int t = tlp ? tlp[r] : -1;
  const int K = t > 0 ? min(min(t, K_max), V) : 0;
  const auto src = row_src<DT>(row, vec, [](float z) { return z != z ? -INFINITY : z; });  // NaN reads as -inf
  auto all = [](float, unsigned int) { return true; };
  auto nomass = [](float) { return 0ull; };

  if (ph == W_SORT) {
    // ---- one workgroup per row: sort the K gathered entries, write them
    int* oid = top_ids + static_cast<size_t>(r) * K_max;
    float* olp = top_lp + static_cast<size_t>(r) * K_max;
    for (int j = K + tid; j < K_max; j += FT) {
      oid[j] = -1;
      olp[j] = -INFINITY;
    }
    if (K == 0) return;
    int np = 1;
    while (np < K) np <<= 1;
    for (int j = tid; j < np; j += FT) sh.ent[j] = j < K ? lst[j] : 0ull;  // padding sorts last
    float M = -INFINITY;
    double S = 0.0;
    for (int q = 0; q < G; ++q) M = fmaxf(M, fr.mxp[q]);
    for (int q = 0; q < G; ++q) S += wr.lsep[q];
    const double lse = static_cast<double>(M) + log(S);
    __syncthreads();
    // each step's np / 2 compare-exchange pairs (i, i | jj), i without bit jj,
    // at most two per thread; both pairs' loads are issued before either store
    // (a step's pairs are disjoint), so a step costs one LDS round trip
    const int npairs = np >> 1;
    for (int k = 2; k <= np; k <<= 1) {
      for (int jj = k >> 1; jj > 0; jj >>= 1) {
        unsigned long long a[2], b[2];
        int ia[2];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const int pr = tid + q * FT;
          ia[q] = ((pr & ~(jj - 1)) << 1) | (pr & (jj - 1));
          if (pr < npairs) {
            a[q] = sh.ent[ia[q]];
            b[q] = sh.ent[ia[q] | jj];
          }
        }
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          if (tid + q * FT < npairs) {
            const bool desc = (ia[q] & k) == 0;
            if (desc ? (a[q] < b[q]) : (a[q] > b[q])) {
              sh.ent[ia[q]] = b[q];
              sh.ent[ia[q] | jj] = a[q];
            }
          }
        }
        __syncthreads();
      }
    }
    for (int j = tid; j < K; j += FT) {
      const unsigned long long e = sh.ent[j];
      const int id = static_cast<int>(0xffffffffu - static_cast<unsigned int>(e));
      oid[j] = id;
      olp[j] = static_cast<float>(static_cast<double>(src.at(id)) - lse);
    }
    return;
  }
  if (K == 0) return;

  if (ph == W_MAX) {
    // ---- the slice max, and the first level of the K-th largest logit
    float mx = -INFINITY;
    row_pass(lo, hi, src, [&](int, float z) { mx = fmaxf(mx, z); });
    const float w = wave_max(mx);
    if ((tid & 63) == 0) sh.f.fr[tid >> 6] = w;
    __syncthreads();
    const float m = rdl(row_max16(sh.f.fr[tid & (FW - 1)]), 0);
    if (tid == 0) {
      fr.mxp[g] = m;
      if (g == 0) wr.n = 0u;
    }
    FSel s{};
    slice_hist<false>(lo, hi, 1, s, src, all, nomass, hcs(0) + g * NBIN, nullptr, sh.f);
    return;
  }
  constexpr int NL = nlev(DT);
  if (ph >= W_K1 && ph <= W_K3) {
    // ---- level l = ph: choose digit l from slot (l - 1) & 1, build level l +
    // 1 into slot l & 1; the first also sums exp(z - M) over the slice
    const int l = ph - W_K1 + 1;
    FSel s{};
    s.rem = s.tgt = static_cast<unsigned long long>(K);
    if (l > 1) s = fr.sk[(l - 1) & 1];
    s = select_level<false, false>(s, l, hcs((l - 1) & 1), nullptr, G, 0.0f, sh.f);
    if (g == 0 && tid == 0) fr.sk[l & 1] = s;
    if (l == 1) {
      float M = -INFINITY;
      for (int q = 0; q < G; ++q) M = fmaxf(M, fr.mxp[q]);
      double part = 0.0;
      slice_hist<false>(lo, hi, 2, s, src, all, nomass, hcs(1) + g * NBIN, nullptr, sh.f,
                        [&](float z) { part += static_cast<double>(wexp(z, M)); });
      const double tot = fsum(part, sh.dr);
      if (tid == 0) wr.lsep[g] = tot;
    } else {
      slice_hist<false>(lo, hi, l + 1, s, src, all, nomass, hcs(l & 1) + g * NBIN, nullptr, sh.f);
    }
    return;
  }
  if (ph == W_TIES) {
    // ---- the last digit: tau is the K-th largest key; each wave segment's
    // count of it
    FSel s = select_level<false, false>(fr.sk[(NL - 1) & 1], NL, hcs((NL - 1) & 1), nullptr, G, 0.0f,
                                        sh.f);
    s.prefix = complete_key<DT>(s.prefix);
    if (g == 0 && tid == 0) fr.sk[NL & 1] = s;
    seg_counts(lo, hi, g, src, [&](float z) { return okey(z) == s.prefix; }, fr.tiec);
    return;
  }

  // ---- W_GATHER: every entry above tau, and the first need_eq of tau's tie
  // group in index order, into LDS, then one reservation of the row's list
  const FSel s = fr.sk[NL & 1];
  const unsigned int tau = s.prefix;
  const unsigned int need_eq = static_cast<unsigned int>(K) - static_cast<unsigned int>(s.abv);
  int s0, s1;
  wave_segment(lo, hi, &s0, &s1);
  if (tid == 0) sh.n = 0u;
  unsigned int rank = segs_before(fr.tiec, g);
  __syncthreads();  // sh.n cleared before the first slot is taken
  seg_pass(s0, s1, src, [&](int i0, const float* v, int n) {
    unsigned int c = 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) c += (e < n && okey(v[e]) == tau) ? 1u : 0u;
    unsigned int tot;
    unsigned int my = rank + lanes_before(c, &tot);
    rank += tot;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (e >= n) continue;
      const unsigned int key = okey(v[e]);
      bool take = key > tau;
      if (key == tau) {
        take = my < need_eq;
        ++my;
      }
      if (take) {
        const unsigned int slot =
            __hip_atomic_fetch_add(&sh.n, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
        const int i = i0 + e;
        if (slot < static_cast<unsigned int>(TOPK_WIDE_MAX))
          sh.ent[slot] = (static_cast<unsigned long long>(key) << 32) | (0xffffffffu - static_cast<unsigned int>(i));
      }
    }
  });
  __syncthreads();
  const unsigned int n = min(sh.n, static_cast<unsigned int>(TOPK_WIDE_MAX));
  if (tid == 0)
    sh.base = n ? __hip_atomic_fetch_add(&wr.n, n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : 0u;
  __syncthreads();
  const unsigned int base = sh.base;
  for (unsigned int j = tid; j < n; j += FT)
    if (base + j < static_cast<unsigned int>(K)) lst[base + j] = sh.ent[j];
}

void set_err(char** err, const std::string& msg) {
  if (!err) return;
  char* q = static_cast<char*>(std::malloc(msg.size() + 1));
  if (q) std::memcpy(q, msg.c_str(), msg.size() + 1);
  *err = q;
}

// Which phases a call launches: every one for per-row parameters, only those
// of the filters that are on for the single-filter calls.
enum FUse { FU_ALL, FU_TOPK, FU_TOPP, FU_MINP };

int launch_filter(const void* d_logits, int dtype, int B, int V, int64_t row_stride, void* d_out, int64_t out_stride,
                  FArgs f, FUse use, void* d_ws, size_t ws_bytes, void* stream, char** err) {
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
  if (!d_ws || ws_bytes < filter_ws_bytes(B, V)) {
    set_err(err, "mlxf: workspace is NULL or smaller than mlxf_filter_workspace_size()");
    return MLXF_EWORKSPACE;
  }
  if (reinterpret_cast<uintptr_t>(d_ws) & 255u) {
    set_err(err, "mlxf: workspace must be 256-byte aligned");
    return MLXF_EINVAL;
  }
  f.logits = d_logits;
  f.row_stride = row_stride;
  f.vec = reinterpret_cast<uintptr_t>(d_logits) % 16 == 0 && (static_cast<size_t>(row_stride) * esz) % 16 == 0;
  f.ovec = reinterpret_cast<uintptr_t>(d_out) % 16 == 0 && (static_cast<size_t>(out_stride) * esz) % 16 == 0;
  f.out = d_out;
  f.out_stride = out_stride;
  f.B = B;
  f.V = V;
  FWs ws;
  ws.G = filter_groups(B, V);
  const size_t nb = static_cast<size_t>(B) * 2 * ws.G * NBIN;
  char* base = static_cast<char*>(d_ws);
  ws.rows = reinterpret_cast<FRow*>(base);
  ws.hc = reinterpret_cast<unsigned int*>(base + fws_align(static_cast<size_t>(B) * sizeof(FRow)));
  ws.hm = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ws.hc) + fws_align(nb * 4));
  int phases[10], np = 0;
  phases[np++] = FP_MAX;
  const int nl = nlev(dtype);
  if (use == FU_ALL || use == FU_TOPK)
    for (int l = 1; l < nl; ++l) phases[np++] = FP_K1 + l - 1;
  if (use != FU_MINP) phases[np++] = FP_P0;
  if (use == FU_ALL || use == FU_TOPP) {
    for (int l = 1; l < nl; ++l) phases[np++] = FP_P1 + l - 1;
    phases[np++] = FP_TIES;
  }
  phases[np++] = FP_FIN;
  hipStream_t st = static_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned int>(B), static_cast<unsigned int>(ws.G)), block(FT);
  for (int q = 0; q < np; ++q) {
    if (dtype == MLXF_DTYPE_F32)
      hipLaunchKernelGGL(k_filter<MLXF_DTYPE_F32>, grid, block, 0, st, f, ws, phases[q]);
    else if (dtype == MLXF_DTYPE_BF16)
      hipLaunchKernelGGL(k_filter<MLXF_DTYPE_BF16>, grid, block, 0, st, f, ws, phases[q]);
    else
      hipLaunchKernelGGL(k_filter<MLXF_DTYPE_F16>, grid, block, 0, st, f, ws, phases[q]);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
      set_err(err, std::string("mlxf: kernel launch failed: ") + hipGetErrorString(e));
      return MLXF_EHIP;
    }
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

size_t topk_wide_ws_bytes(int B, int V, int K_max) { return K_max > TOPK_LIST ? wide_ws_bytes(B, V, K_max) : 0; }

hipError_t launch_topk_wide(const void* logits, int dtype, int B, int V, long long row_stride, const int* tlp,
                            int K_max, int* top_ids, float* top_lp, void* d_ws, hipStream_t st) {
  WWs ws;
  ws.G = filter_groups(B, V);
  const size_t nb = static_cast<size_t>(B) * 2 * ws.G * NBIN;
  char* base = static_cast<char*>(d_ws);
  ws.rows = reinterpret_cast<WRow*>(base);
  ws.hc = reinterpret_cast<unsigned int*>(base + fws_align(static_cast<size_t>(B) * sizeof(WRow)));
  ws.list = reinterpret_cast<unsigned long long*>(reinterpret_cast<char*>(ws.hc) + fws_align(nb * 4));
  const size_t esz = dtype == MLXF_DTYPE_F32 ? 4 : 2;
  const bool vec = reinterpret_cast<uintptr_t>(logits) % 16 == 0 && (static_cast<size_t>(row_stride) * esz) % 16 == 0;
  const int nl = nlev(dtype);
  for (int ph = W_MAX; ph <= W_SORT; ++ph) {
    if (ph >= W_K1 && ph <= W_K3 && ph - W_K1 + 1 >= nl) continue;  // levels the dtype does not need
    const dim3 grid(static_cast<unsigned int>(B), ph == W_SORT ? 1u : static_cast<unsigned int>(ws.G)), block(FT);
    if (dtype == MLXF_DTYPE_F32)
      hipLaunchKernelGGL(k_topk_wide<MLXF_DTYPE_F32>, grid, block, 0, st, logits, row_stride, V, tlp, K_max, top_ids,
                         top_lp, ws, ph, vec);
    else if (dtype == MLXF_DTYPE_BF16)
      hipLaunchKernelGGL(k_topk_wide<MLXF_DTYPE_BF16>, grid, block, 0, st, logits, row_stride, V, tlp, K_max, top_ids,
                         top_lp, ws, ph, vec);
    else
      hipLaunchKernelGGL(k_topk_wide<MLXF_DTYPE_F16>, grid, block, 0, st, logits, row_stride, V, tlp, K_max, top_ids,
                         top_lp, ws, ph, vec);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace mlxf

extern "C" int mlxf_filter_workspace_size(int B, int V, size_t* bytes, char** err) {
  if (!bytes || B < 0 || V < 1 || V > MLXF_MAX_VOCAB) {
    mlxf::set_err(err, "mlxf: bad arguments (bytes non-NULL, B >= 0, V in [1, MLXF_MAX_VOCAB])");
    return MLXF_EINVAL;
  }
  *bytes = B == 0 ? 0 : mlxf::filter_ws_bytes(B, V);
  return MLXF_OK;
}

extern "C" int mlxf_filter_logits(const void* d_logits, int dtype, int B, int V, int64_t row_stride,
                                  const float* d_temperature, const int32_t* d_top_k, const float* d_top_p,
                                  const float* d_min_p, void* d_out, int64_t out_stride, void* d_workspace,
                                  size_t workspace_bytes, void* stream, char** err) {
  try {
    mlxf::FArgs f = mlxf::scalars(0.0f, 0, 1.0f, 0.0f);
    f.T = d_temperature;
    f.k = d_top_k;
    f.p = d_top_p;
    f.minp = d_min_p;
    return mlxf::launch_filter(d_logits, dtype, B, V, row_stride, d_out, out_stride, f, mlxf::FU_ALL, d_workspace,
                               workspace_bytes, stream, err);
  } catch (...) {
    mlxf::set_err(err, "mlxf: unexpected exception");
    return MLXF_EINVAL;
  }
}

extern "C" int mlxf_apply_top_k(const void* d_logits, int dtype, int B, int V, int64_t row_stride, int k,
                                void* d_out, int64_t out_stride, void* d_workspace, size_t workspace_bytes,
                                void* stream, char** err) {
  return mlxf::launch_filter(d_logits, dtype, B, V, row_stride, d_out, out_stride, mlxf::scalars(0.0f, k, 1.0f, 0.0f),
                             mlxf::FU_TOPK, d_workspace, workspace_bytes, stream, err);
}

extern "C" int mlxf_apply_top_p(const void* d_logits, int dtype, int B, int V, int64_t row_stride, float p,
                                void* d_out, int64_t out_stride, void* d_workspace, size_t workspace_bytes,
                                void* stream, char** err) {
  return mlxf::launch_filter(d_logits, dtype, B, V, row_stride, d_out, out_stride, mlxf::scalars(0.0f, 0, p, 0.0f),
                             mlxf::FU_TOPP, d_workspace, workspace_bytes, stream, err);
}

extern "C" int mlxf_apply_min_p(const void* d_logits, int dtype, int B, int V, int64_t row_stride, float min_p,
                                void* d_out, int64_t out_stride, void* d_workspace, size_t workspace_bytes,
                                void* stream, char** err) {
  return mlxf::launch_filter(d_logits, dtype, B, V, row_stride, d_out, out_stride,
                             mlxf::scalars(0.0f, 0, 1.0f, min_p), mlxf::FU_MINP, d_workspace, workspace_bytes,
                             stream, err);
}
