#pragma once
// rowhist.hpp -- the row-histogram path for bf16 logits: one 1024-thread
// workgroup per row reads the row once and counts it into exact per-value
// histograms in LDS, from which every selection of Sampler::sample
// (src/sample/sampler.cpp:141-166) follows without touching the logits
// again; only the draw re-reads an eighth (a quarter with split counting) of
// the row.
//
// Why it is exact: for bf16 logits, z' = round_bf16(z / T), the weight
// w = exp2(fma(z', log2 e, -RN(max z' log2 e))) and its fixed-point mass
// floor(w 2^40) are functions of the 16-bit value alone.  So the count of
// each distinct value is all the top-k count, the nucleus mass and min_p need:
// a bin's mass is count x mass(value), an exact integer, and every cutoff is
// found on the bins with the same integers the per-element path sums.
//
// Bins.  A bin is one bf16 value with magnitude in [2^-28, 2^8) (36 binades of
// 128 values per sign), plus three merged bins: |z| < 2^-28 ("tiny", which
// holds +-0), z <= -256 (with -inf and negative NaNs) and z >= 256 (with +inf
// and positive NaNs).  A merged bin has one weight only when its elements'
// z' cannot be told apart by the weight function: the tiny bin when |z' log2 e|
// stays below half an ulp of the weight's offset, the low bin when its weight
// rounds to a zero mass.  The row is split into four contiguous chunks with a
// histogram each (4 x 9220 32-bit counter words, 144 KB of LDS), so per-chunk
// kept masses locate the draw to one chunk, which the walk then reads.  When
// the workgroup counts its row itself, each word holds two 16-bit counters,
// one for each half of its chunk, and the walk reads one of eight half chunks
// (at most 65535 logits each: V <= 458752); with split counting (chunk
// workgroups, few rows) the counters are 32-bit and the walk reads a chunk.
//
// Rows the bins cannot decide exactly -- the maximum in a merged bin (a
// logit >= 256, +inf, a positive NaN, or a row of values all within 2^-28 of
// zero or below -256), a cutoff that falls in or next to a merged bin, or a
// merged bin whose elements' weights differ -- fall back to the per-slice
// path in the same workgroup: its first four waves run the first pass over
// the row's slices and the deciding step (every refine level), the other
// twelve end.
//
// Memory per row: one read of the row (V * 2 bytes) in pass 1, a half chunk
// (or a chunk) in the draw.  No MFMA: nothing here is a dense contraction.

namespace mlxf {

// Per-call constants of the row-histogram path.
struct RhArgs {
  int ipc;                   // pass-1 iterations per chunk (chunk length ipc * 8192 logits;
                             // even when the counters are packed)
  int nfull;                 // iterations wholly inside the row
  // split calls (few rows): one workgroup per chunk counts it into
  // hsplit[r][c][bin]; crec[r][c] = (largest bin offset + 65536) | lowest
  // index holding it << 32 (the index only for greedy rows)
  unsigned int* hsplit;
  unsigned long long* crec;
};

// One bf16 call on the row-histogram path (defined in sampler_bf16.hip).
hipError_t launch_row16_bf16(const Args& a, int ept, const RhArgs& x, hipStream_t st);

// Per-phase timestamps for a profiling harness that defines MLXF_RH_STAMPS
// (and the array it writes); no effect otherwise.
#ifdef MLXF_RH_STAMPS
#define MLXF_RH_STAMP(i) \
  if (threadIdx.x == 0) mlxf_rh_stamps[blockIdx.x * 16 + (i)] = __builtin_amdgcn_s_memrealtime()
#define MLXF_RH_WSTAMP(i) \
  if ((threadIdx.x & 63) == 0) mlxf_rh_stamps[16384 + (blockIdx.x * 16 + (threadIdx.x >> 6)) * 16 + (i)] = __builtin_amdgcn_s_memrealtime()
#define MLXF_RC_STAMP(i) \
  if (threadIdx.x == 0) mlxf_rh_stamps[8192 + blockIdx.x * 8 + (i)] = __builtin_amdgcn_s_memrealtime()
#else
#define MLXF_RH_STAMP(i)
#define MLXF_RH_WSTAMP(i)
#define MLXF_RC_STAMP(i)
#endif

namespace {
namespace rh {

constexpr int NT = 1024;             // threads per workgroup (16 waves, 4 per SIMD)
constexpr int NWV = NT / 64;
constexpr int NWIN = 4608;           // bf16 magnitudes in [2^-28, 2^8): 36 binades x 128
constexpr int LOMAG = 0x3180;        // bf16 bit pattern of 2^-28
constexpr int NBIN = 2 * NWIN + 3;   // window bins of both signs + three merged bins
constexpr int B_NEGHUGE = 0;         // z <= -256, -inf, negative NaN
constexpr int B_TINY = NWIN + 1;     // |z| < 2^-28, +-0
constexpr int B_POSHUGE = 2 * NWIN + 2;  // z >= 256, +inf, positive NaN
constexpr int B_TRASH = NBIN;        // elements past the row end
constexpr int CHW = NBIN + 1;        // counters per chunk histogram
constexpr int CHB = CHW * 4;         // bytes per chunk histogram (36880)
constexpr int NCH = 4;               // chunk histograms per row
constexpr int NSUB_MAX = 8;          // chunks the walk picks from: the halves of the four (packed
                                     // counters) when one workgroup counts the row, else the four
constexpr int ITER = NT * 8;         // elements one pass-1 iteration covers
constexpr int BPT = 11;              // bins per thread in the deciding step (11 * 1024 >= NBIN;
                                     // an odd stride keeps a wave's LDS accesses on distinct banks)
// LDS: chunk c's histogram at byte c * CHB.  Pass 1 addresses a counter as
// page + immediate + 4 * bin with 16-bit packed bin offsets: chunks 0 and 1 on
// page 0 (immediates 0 and CHB), chunks 2 and 3 on page 65536 with the
// offsets raised by 2 * CHB - 65536.
constexpr unsigned PAGE1 = 65536u;
constexpr unsigned PAGE1_ADD = 2u * CHB - PAGE1;
constexpr size_t HIST_BYTES = static_cast<size_t>(NCH) * CHB;

typedef short s16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int SPARSE = 512;  // largest sparse draw list (elements at or above the cutoff in the chunk)
struct Scratch {
  unsigned long long u64r[NWV][NSUB_MAX];
  double dr[NWV];
  unsigned long long ugn[NWV][NSUB_MAX];
  unsigned int lst[SPARSE];
  int ir[NWV][2];
  unsigned long long sel64[8];
  int sel[16];
};
constexpr size_t LDS_BYTES = HIST_BYTES + sizeof(Scratch);
static_assert(LDS_BYTES <= 160 * 1024, "row-histogram LDS exceeds a CU's 160 KB");

// Bin offsets of the two bf16 values of a 32-bit word, packed signed 16-bit:
// x = t for a positive value and -t for a negative one, t = clamp(magnitude
// bits - LOMAG + 1, 0, NWIN + 1) (t = 0: tiny, t = NWIN + 1: beyond the
// window); the bin is NWIN + 1 + x.  Monotone non-decreasing in the value.
__device__ __forceinline__ unsigned int binx2(unsigned int w) {
  u16x2 t = __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, w & 0x7fff7fffu),
                                          (u16x2){static_cast<unsigned short>(LOMAG - 1), static_cast<unsigned short>(LOMAG - 1)});
  t = __builtin_elementwise_min(t, (u16x2){static_cast<unsigned short>(NWIN + 1), static_cast<unsigned short>(NWIN + 1)});
  const s16x2 sg = __builtin_bit_cast(s16x2, w) >> (s16x2){15, 15};
  return __builtin_bit_cast(unsigned int, (__builtin_bit_cast(s16x2, t) ^ sg) - sg);
}
// The bins themselves, packed.
__device__ __forceinline__ unsigned int bins2(unsigned int w) {
  return __builtin_bit_cast(unsigned int, __builtin_bit_cast(s16x2, binx2(w)) +
                                              (s16x2){static_cast<short>(NWIN + 1), static_cast<short>(NWIN + 1)});
}
__device__ __forceinline__ unsigned int pkmax_i16(unsigned int a, unsigned int b) {
  return __builtin_bit_cast(unsigned int,
                            __builtin_elementwise_max(__builtin_bit_cast(s16x2, a), __builtin_bit_cast(s16x2, b)));
}

__device__ __forceinline__ unsigned int pkmax_u16(unsigned int a, unsigned int b) {
  return __builtin_bit_cast(unsigned int,
                            __builtin_elementwise_max(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}

// The bf16 value of a window bin (merged bins: a representative).
__device__ __forceinline__ float bin_value(int b) {
  if (b >= 1 && b <= NWIN) return __uint_as_float((0x8000u | static_cast<unsigned>(LOMAG + NWIN - b)) << 16);
  if (b >= NWIN + 2 && b <= 2 * NWIN + 1) return __uint_as_float(static_cast<unsigned>(LOMAG + b - (NWIN + 2)) << 16);
  if (b == B_TINY) return 0.0f;
  return b == B_POSHUGE ? INFINITY : -INFINITY;
}

// Bin owned by thread tid at slot j of the deciding step: bins in descending
// order from the top, BPT per thread; negative = none.
__device__ __forceinline__ int own_bin(int tid, int j) { return NBIN - 1 - (tid * BPT + j); }

// ---- block primitives for NT threads (16 waves).  The 16 per-wave values
// are combined by lanes 0..15 of every wave (one LDS read each and a 4-step
// row reduction), not by a loop in every thread: at 16 waves on 4 SIMDs each
// VALU instruction of a thread costs 16 cycles of a SIMD.
static_assert(NWV == 16, "the wave combine is one row of 16 lanes");
template <typename T>
__device__ __forceinline__ T bsum(T x, T* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  x = wave_sum(x);
  __syncthreads();
  if (lane == 0) red[wid] = x;
  __syncthreads();
  return rdl(row_sum16(lane < NWV ? red[lane & (NWV - 1)] : T(0)), 0);
}
__device__ __forceinline__ int bmin_i(int x, int* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  x = wave_min(x);
  __syncthreads();
  if (lane == 0) red[wid] = x;
  __syncthreads();
  return rdl(row_min16(red[lane & (NWV - 1)]), 0);
}
__device__ __forceinline__ int bmax_i(int x, int* red) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  x = wave_max(x);
  __syncthreads();
  if (lane == 0) red[wid] = x;
  __syncthreads();
  return rdl(row_max16(red[lane & (NWV - 1)]), 0);
}
// Exclusive scan over threads in index order; *total = the block sum.
template <typename T>
__device__ __forceinline__ T bscan(T x, T* red, T* total) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const T inc = wave_incl_scan_dpp(x);
  __syncthreads();
  if (lane == 63) red[wid] = inc;
  __syncthreads();
  const T ws = row_incl_scan16(lane < NWV ? red[lane & (NWV - 1)] : T(0));
  *total = rdl(ws, NWV - 1);
  const T before = rdl(ws, wid > 0 ? wid - 1 : 0);
  return inc - x + (wid > 0 ? before : T(0));
}

// bscan of a 64-bit x and an int y at once (one pair of barriers): the
// exclusive scans are returned in *ex, *ey, the block sums in *tx, *ty.
__device__ __forceinline__ void bscan2(unsigned long long x, int y, unsigned long long* redx, int* redy,
                                       unsigned long long* ex, int* ey, unsigned long long* tx, int* ty) {
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  const unsigned long long ix = wave_incl_scan_dpp(x);
  const int iy = wave_incl_scan_dpp(y);
  __syncthreads();
  if (lane == 63) {
    redx[wid] = ix;
    redy[wid] = iy;
  }
  __syncthreads();
  const unsigned long long wx = row_incl_scan16(lane < NWV ? redx[lane & (NWV - 1)] : 0ull);
  const int wy = row_incl_scan16(lane < NWV ? redy[lane & (NWV - 1)] : 0);
  *tx = rdl(wx, NWV - 1);
  *ty = rdl(wy, NWV - 1);
  const int src = wid > 0 ? wid - 1 : 0;
  const unsigned long long bx = rdl(wx, src);
  const int by = rdl(wy, src);
  *ex = ix - x + (wid > 0 ? bx : 0ull);
  *ey = iy - y + (wid > 0 ? by : 0);
}

// ---- pass 1: one word (two values, as bin offsets x2) into chunk histogram
// (PAGE, ADD, IMM); inc is 1, or 65536 for the second half of a chunk with
// packed counters
template <unsigned PAGE, unsigned ADD, unsigned IMM>
__device__ __forceinline__ void count_word(unsigned char* lds, unsigned int x2, unsigned int inc) {
  constexpr unsigned short K = static_cast<unsigned short>(4u * (NWIN + 1) + ADD);
  const u16x2 o = __builtin_bit_cast(u16x2, x2) * (u16x2){4, 4} + (u16x2){K, K};
  const unsigned int o2 = __builtin_bit_cast(unsigned int, o);
  // page 1: the low half's address takes its top bytes from PAGE by a byte
  // permute (one operation, and IMM stays in the instruction's offset field)
  const unsigned int a0 = PAGE ? __builtin_amdgcn_perm(PAGE, o2, 0x07060100u) : (o2 & 0xffffu);
  const unsigned int a1 = PAGE ? __builtin_amdgcn_alignbit(PAGE >> 16, o2, 16) : (o2 >> 16);
  atomicAdd(reinterpret_cast<unsigned int*>(lds + IMM + a0), inc);
  atomicAdd(reinterpret_cast<unsigned int*>(lds + IMM + a1), inc);
}

// One iteration (8 values) into a chunk histogram; best / bestit track the
// largest bin offset and the first iteration holding it.
template <unsigned PAGE, unsigned ADD, unsigned IMM>
__device__ __forceinline__ void count_iter(unsigned char* lds, const uint4& q, int it, unsigned int inc, int& best,
                                           int& bestit) {
  const unsigned int w[4] = {q.x, q.y, q.z, q.w};
  unsigned int m = 0x80008000u;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const unsigned int x2 = binx2(w[k]);
    m = pkmax_i16(m, x2);
    count_word<PAGE, ADD, IMM>(lds, x2, inc);
  }
  const int mf = max(static_cast<int>(static_cast<short>(m & 0xffffu)), static_cast<int>(static_cast<short>(m >> 16)));
  if (mf > best) {
    best = mf;
    bestit = it;
  }
}

// One iteration into the histogram of chunk c (wave-uniform).
__device__ __forceinline__ void count_iter_c(unsigned char* lds, const uint4& q, int it, int c, unsigned int inc,
                                             int& best, int& bestit) {
  if (c == 0)
    count_iter<0u, 0u, 0u>(lds, q, it, inc, best, bestit);
  else if (c == 1)
    count_iter<0u, 0u, static_cast<unsigned>(CHB)>(lds, q, it, inc, best, bestit);
  else if (c == 2)
    count_iter<PAGE1, PAGE1_ADD, 0u>(lds, q, it, inc, best, bestit);
  else
    count_iter<PAGE1, PAGE1_ADD, static_cast<unsigned>(CHB)>(lds, q, it, inc, best, bestit);
}

// This thread's word of the iteration the row ends in (ITER * it < V <
// ITER * (it + 1)): a vector load when its 8 elements are all in the row,
// element by element for the one word holding the row end, zeros past it.
__device__ __forceinline__ uint4 tail_word(const unsigned short* row, int V, int it) {
  const int p0 = it * ITER + static_cast<int>(threadIdx.x) * 8;
  if (p0 + 8 <= V) return reinterpret_cast<const uint4*>(row)[static_cast<size_t>(it) * NT + threadIdx.x];
  unsigned int w[4] = {0u, 0u, 0u, 0u};
  if (p0 < V) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const unsigned int lo = p0 + 2 * k < V ? row[p0 + 2 * k] : 0u;
      const unsigned int hi = p0 + 2 * k + 1 < V ? row[p0 + 2 * k + 1] : 0u;
      w[k] = lo | (hi << 16);
    }
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Counts the tail word q (from tail_word).  A thread wholly past the end
// counts nothing (all its elements in one counter would serialise the wave's
// atomics); past-the-end elements of the word holding the end count in the
// trash slot and not towards the maximum.
__device__ __forceinline__ void count_tail(unsigned char* lds, const uint4& q, int V, int it, int c,
                                           unsigned int inc, int& best, int& bestit) {
  const int p0 = it * ITER + static_cast<int>(threadIdx.x) * 8;
  if (p0 >= V) return;
  const unsigned int w[4] = {q.x, q.y, q.z, q.w};
  constexpr unsigned int XT = static_cast<unsigned>(B_TRASH - (NWIN + 1));
  int mf = -32768;
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    unsigned int x2 = binx2(w[k]);
    const bool vlo = p0 + 2 * k < V, vhi = p0 + 2 * k + 1 < V;
    if (vlo) mf = max(mf, static_cast<int>(static_cast<short>(x2 & 0xffffu)));
    if (vhi) mf = max(mf, static_cast<int>(static_cast<short>(x2 >> 16)));
    x2 = (vlo ? (x2 & 0xffffu) : XT) | (vhi ? (x2 & 0xffff0000u) : (XT << 16));
    if (c == 0)
      count_word<0u, 0u, 0u>(lds, x2, inc);
    else if (c == 1)
      count_word<0u, 0u, static_cast<unsigned>(CHB)>(lds, x2, inc);
    else if (c == 2)
      count_word<PAGE1, PAGE1_ADD, 0u>(lds, x2, inc);
    else
      count_word<PAGE1, PAGE1_ADD, static_cast<unsigned>(CHB)>(lds, x2, inc);
  }
  if (mf > best) {
    best = mf;
    bestit = it;
  }
}

// Pass 1 over the whole row: D iterations' loads in flight (a register ring;
// the first D are issued before the histograms are cleared, so the clear
// overlaps them), chunk c = it / ipc; with packed counters (PK, ipc even) the
// second half of a chunk's iterations counts in the high 16 bits.
template <int D, bool PK>
__device__ __forceinline__ void count_row(unsigned char* lds, const unsigned short* row, int V, int ipc, int nfull,
                                          int& best, int& bestit) {
  const int tid = threadIdx.x;
  const uint4* rv = reinterpret_cast<const uint4*>(row);
  const bool has_tail = nfull * ITER < V;
  uint4 tq = make_uint4(0u, 0u, 0u, 0u);
  if (has_tail) tq = tail_word(row, V, nfull);  // requested first: its latency hides behind the row
  uint4 buf[D];
#pragma unroll
  for (int j = 0; j < D; ++j)
    if (j < nfull) buf[j] = rv[static_cast<size_t>(j) * NT + tid];
  {
    uint4* h4 = reinterpret_cast<uint4*>(lds);
    for (int i = tid; i < NCH * CHW / 4; i += NT) h4[i] = make_uint4(0u, 0u, 0u, 0u);
  }
  __syncthreads();
  for (int it = 0; it < nfull; it += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int i = it + j;
      if (i < nfull) {
        const uint4 q = buf[j];
        if (i + D < nfull) buf[j] = rv[static_cast<size_t>(i + D) * NT + tid];
        const int c = (i >= ipc) + (i >= 2 * ipc) + (i >= 3 * ipc);
        const unsigned int inc = PK && i - c * ipc >= (ipc >> 1) ? 0x10000u : 1u;
        count_iter_c(lds, q, i, c, inc, best, bestit);
      }
    }
  }
  if (has_tail) {
    const int c = (nfull >= ipc) + (nfull >= 2 * ipc) + (nfull >= 3 * ipc);
    const unsigned int inc = PK && nfull - c * ipc >= (ipc >> 1) ? 0x10000u : 1u;
    count_tail(lds, tq, V, nfull, c, inc, best, bestit);
  }
}

// Pass 1 over one chunk (iterations [it0, it1), plus the row's last partial
// iteration when has_tail) into the histogram at the start of lds; the same
// register ring as count_row.
template <int D>
__device__ __forceinline__ void count_chunk(unsigned char* lds, const unsigned short* row, int V, int it0, int it1,
                                            bool has_tail, int& best, int& bestit) {
  const int tid = threadIdx.x;
  const uint4* rv = reinterpret_cast<const uint4*>(row);
  uint4 tq = make_uint4(0u, 0u, 0u, 0u);
  if (has_tail) tq = tail_word(row, V, it1);
  uint4 buf[D];
#pragma unroll
  for (int j = 0; j < D; ++j)
    if (it0 + j < it1) buf[j] = rv[static_cast<size_t>(it0 + j) * NT + tid];
  {
    uint4* h4 = reinterpret_cast<uint4*>(lds);
    for (int i = tid; i < CHW / 4; i += NT) h4[i] = make_uint4(0u, 0u, 0u, 0u);
  }
  __syncthreads();
  for (int it = it0; it < it1; it += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int i = it + j;
      if (i < it1) {
        const uint4 q = buf[j];
        if (i + D < it1) buf[j] = rv[static_cast<size_t>(i + D) * NT + tid];
        count_iter<0u, 0u, 0u>(lds, q, i, 1u, best, bestit);
      }
    }
  }
  if (has_tail) count_tail(lds, tq, V, it1, 0, 1u, best, bestit);
}

// Lowest index in this thread's 8 elements of iteration it whose bin is b
// (INT_MAX if none).
__device__ __forceinline__ int first_at(const unsigned short* row, int V, int it, int b) {
  int myarg = INT_MAX;
  const int p0 = it * ITER + static_cast<int>(threadIdx.x) * 8;
  for (int j = 0; j < 8 && myarg == INT_MAX; j += 2) {
    const unsigned int lo = p0 + j < V ? row[p0 + j] : 0u;
    const unsigned int hi = p0 + j + 1 < V ? row[p0 + j + 1] : 0u;
    const unsigned int b2 = bins2(lo | (hi << 16));
    if (p0 + j < V && static_cast<int>(b2 & 0xffffu) == b)
      myarg = p0 + j;
    else if (p0 + j + 1 < V && static_cast<int>(b2 >> 16) == b)
      myarg = p0 + j + 1;
  }
  return myarg;
}

// Counts with packed counters (PK): the word of chunk c holds the count of its
// first half (the walk's chunk 2c) in the low 16 bits and of its second half
// (chunk 2c + 1) in the high 16 bits.  hsub: walk chunk c's count of bin b;
// htot: the row's count of bin b.
template <bool PK>
__device__ __forceinline__ unsigned int hsub(const unsigned int* hist, int c, int b) {
  if constexpr (PK) {
    const unsigned int w = hist[(c >> 1) * CHW + b];
    return (c & 1) ? (w >> 16) : (w & 0xffffu);
  } else {
    return hist[c * CHW + b];
  }
}
template <bool PK>
__device__ __forceinline__ unsigned int htot(const unsigned int* hist, int b) {
  const unsigned int w0 = hist[b], w1 = hist[CHW + b], w2 = hist[2 * CHW + b], w3 = hist[3 * CHW + b];
  if constexpr (PK)
    return ((w0 & 0xffffu) + (w0 >> 16)) + ((w1 & 0xffffu) + (w1 >> 16)) + ((w2 & 0xffffu) + (w2 >> 16)) +
           ((w3 & 0xffffu) + (w3 >> 16));
  else
    return (w0 + w1) + (w2 + w3);
}

// Wave reduce-scatter of N per-lane values (N = 4 or 8): lane l receives the
// wave's sum of v[l / (64 / N)].  Each step halves the values a lane holds,
// swapping the other half with the lane 32, 16 (and 8) places away; the
// remaining lanes of a group then sum by exchanges (whole wave active).
// Lane src's value (ds_bpermute; whole wave active).
__device__ __forceinline__ unsigned long long shfl_u64(unsigned long long v, int src) {
  const int lo = __shfl(static_cast<int>(v), src, 64), hi = __shfl(static_cast<int>(v >> 32), src, 64);
  return (static_cast<unsigned long long>(static_cast<unsigned int>(hi)) << 32) | static_cast<unsigned int>(lo);
}
template <int M, typename T>
__device__ __forceinline__ T rs_step(T a, T b) {
  const bool up = (threadIdx.x & M) != 0;
  return (up ? b : a) + xshf<M>(up ? a : b);
}
template <int N, typename T>
__device__ __forceinline__ T wave_rs(const T (&v)[N]) {
  static_assert(N == 4 || N == 8, "four or eight values");
  T a[N / 2];
#pragma unroll
  for (int i = 0; i < N / 2; ++i) a[i] = rs_step<32>(v[i], v[N / 2 + i]);
  T b[N / 4];
#pragma unroll
  for (int i = 0; i < N / 4; ++i) b[i] = rs_step<16>(a[i], a[N / 4 + i]);
  T c;
  if constexpr (N == 8) {
    c = rs_step<8>(b[0], b[1]);
  } else {
    c = b[0];
    c += xshf<8>(c);
  }
  c += xshf<4>(c);
  c += xshf<2>(c);
  c += xshf<1>(c);
  return c;
}

// The row's kept set after top-k, top-p and min_p, on the bins: every bin
// >= kb whole, plus (when t > 0) the first t elements in index order of the
// tie group [glo, ghi] (one z' value) below it.
struct Kept {
  int kb, glo, ghi;
  unsigned int t;
  unsigned long long wt;
};

// The walk's per-thread sum over its EPTW consecutive elements from c0: the
// kept mass from the weight table (low 56 bits; masses stay far below 2^56:
// at most 128 elements of at most 2^41 each), and with PARTIAL the count
// of the partial tie group's elements (top 8 bits; at most 128 per thread).
// The first WG 16-byte words come preloaded (requested before the weight
// table was built).
template <bool PARTIAL, int WG>
__device__ __forceinline__ unsigned long long walk_sum(const unsigned short* row, int V, int c0, int EPTW,
                                                       const unsigned long long* tab, const Kept& kp,
                                                       const uint4 (&wq0)[WG], bool whole) {
  unsigned long long km = 0ull;
  int gt = 0;
  const unsigned int span = static_cast<unsigned>(kp.ghi - kp.glo);
  auto add_word = [&](unsigned int b2) {
    const unsigned int b0 = b2 & 0xffffu, b1 = b2 >> 16;
    km += tab[b0] + tab[b1];
    if (PARTIAL) gt += (b0 - static_cast<unsigned>(kp.glo) <= span ? 1 : 0) + (b1 - static_cast<unsigned>(kp.glo) <= span ? 1 : 0);
  };
  if (whole) {
    // the first WG words came preloaded; the rest (long rows) in groups
    const uint4* rv = reinterpret_cast<const uint4*>(row + c0);
#pragma unroll
    for (int k = 0; k < WG; ++k) {
      if (k < EPTW / 8) {
        add_word(bins2(wq0[k].x));
        add_word(bins2(wq0[k].y));
        add_word(bins2(wq0[k].z));
        add_word(bins2(wq0[k].w));
      }
    }
    for (int g0 = WG; g0 < EPTW / 8; g0 += WG) {
      uint4 wq[WG];
#pragma unroll
      for (int k = 0; k < WG; ++k)
        if (g0 + k < EPTW / 8) wq[k] = rv[g0 + k];
#pragma unroll
      for (int k = 0; k < WG; ++k) {
        if (g0 + k < EPTW / 8) {
          add_word(bins2(wq[k].x));
          add_word(bins2(wq[k].y));
          add_word(bins2(wq[k].z));
          add_word(bins2(wq[k].w));
        }
      }
    }
  } else {
    // the row ends in this thread's range: element by element
    for (int e = 0; e < EPTW; e += 2) {
      const int p = c0 + e;
      const unsigned int lo = p < V ? row[p] : 0u;
      const unsigned int hi = p + 1 < V ? row[p + 1] : 0u;
      unsigned int b2 = bins2(lo | (hi << 16));
      if (p >= V) b2 = (b2 & 0xffff0000u) | static_cast<unsigned>(B_TRASH);
      if (p + 1 >= V) b2 = (b2 & 0xffffu) | (static_cast<unsigned>(B_TRASH) << 16);
      add_word(b2);
    }
  }
  return km | (static_cast<unsigned long long>(gt) << 56);
}

}  // namespace rh

// The fallback, out of line: its register demand (the deciding step's) stays
// out of the histogram path's register allocation; the LDS pointer keeps its
// address space, so its accesses stay LDS instructions.
// The call's arguments are read from the kernel's argument segment (a copy
// would be a stack frame for every wave).
template <int DT, int EPT>
__device__ __noinline__ void row_fallback(__attribute__((address_space(4))) const Args* ka, int r,
                                          __attribute__((address_space(3))) unsigned char* lds3) {
  const Args& a = *(const Args*)ka;
  FbShared& fsh = *reinterpret_cast<FbShared*>((unsigned char*)lds3);
  for (int s = 0; s < a.S; ++s) {
    scan1_slice<DT, EPT, true>(a, r, s, fsh.s1);
    __syncthreads();
  }
  // the slice records and lists this workgroup wrote are complete; drop stale
  // L1 lines before reading them back
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  decide1_row<DT, EPT, true>(a, r, 0, fsh.d1);
}

constexpr int RH_DEPTH = 6;  // pass-1 iterations in flight per thread (96 KB per workgroup)

// Split calls, first kernel: workgroup (r, c) counts chunk c of row r into
// hsplit[r][c] and records the chunk's largest bin (and, for a greedy row, the
// lowest index holding it) in crec[r][c].  Workgroup ids are laid out so that
// a row's four chunks and its deciding workgroup (k_row16, id r) share an XCD
// (id mod 8 = r mod 8).
template <int DT>
__global__ __launch_bounds__(rh::NT, 1) void k_cnt16(Args a, RhArgs x) {
  using namespace rh;
  __shared__ __align__(16) unsigned char lds[CHB];
  __shared__ int red[NWV];
  const int tid = threadIdx.x;
  const int id = static_cast<int>(blockIdx.x);
  const int grp = id / (8 * NCH), rem = id - grp * (8 * NCH);
  const int c = rem >> 3, r = grp * 8 + (rem & 7);
  if (r >= a.B) return;
  const int V = a.V;
  const Mode md = decode<DT>(a, r);
  const unsigned short* row = static_cast<const unsigned short*>(row_ptr<DT>(a, r));
  // chunk c: iterations [c * ipc, (c + 1) * ipc) of the nfull whole ones, and
  // the partial last iteration (index nfull) when it falls in this chunk
  const int it0 = min(c * x.ipc, x.nfull), it1 = min((c + 1) * x.ipc, x.nfull);
  const bool has_tail = x.nfull * ITER < V && x.nfull >= c * x.ipc && x.nfull < (c + 1) * x.ipc;
  int best = -(NWIN + 1) - 1;
  int bestit = -1;
  MLXF_RC_STAMP(0);
  count_chunk<RH_DEPTH>(lds, row, V, it0, it1, has_tail, best, bestit);
  __syncthreads();
  MLXF_RC_STAMP(1);
  const int cmax = bmax_i(best, red);  // bin offset; -(NWIN + 2) for an empty chunk
  int cid = INT_MAX;
  if (!md.sampling) {
    const int myarg = best == cmax && bestit >= 0 ? first_at(row, V, bestit, cmax + NWIN + 1) : INT_MAX;
    cid = bmin_i(myarg, red);
  }
  MLXF_RC_STAMP(2);
  uint4* dst = reinterpret_cast<uint4*>(x.hsplit + (static_cast<size_t>(r) * NCH + c) * CHW);
  const uint4* src = reinterpret_cast<const uint4*>(lds);
  for (int i = tid; i < CHW / 4; i += NT) dst[i] = src[i];
  MLXF_RC_STAMP(3);
  if (tid == 0)
    x.crec[r * NCH + c] = static_cast<unsigned long long>(static_cast<unsigned>(cmax + 65536)) |
                          (static_cast<unsigned long long>(static_cast<unsigned>(cid)) << 32);
}

// SPLIT: the row's chunk histograms come from k_cnt16 (loaded into the LDS
// layout pass 1 builds), the row maximum and a greedy row's index from its
// chunk records; otherwise pass 1 counts the whole row here.
template <int DT, int EPT, bool SPLIT>
__global__ __launch_bounds__(rh::NT, 1) void k_row16(Args a, RhArgs x) {
  using namespace rh;
  // counting here, the counters are packed and the walk picks one of eight
  // half chunks; with split counting, one of the four chunks
  constexpr bool PK = !SPLIT;
  constexpr int NSUB = PK ? 2 * NCH : NCH;
  __shared__ __align__(16) unsigned char lds[LDS_BYTES];
  unsigned int* hist = reinterpret_cast<unsigned int*>(lds);
  Scratch& sc = *reinterpret_cast<Scratch*>(lds + HIST_BYTES);
  const int tid = threadIdx.x, lane = tid & 63;
  const int r = static_cast<int>(blockIdx.x);
  const int V = a.V;
  const Mode md = decode<DT>(a, r);
  const unsigned short* row = static_cast<const unsigned short*>(row_ptr<DT>(a, r));

  MLXF_RH_STAMP(0);
  int bmax;
  int id = -1;
  bool fb;
  if constexpr (SPLIT) {
    static_assert(HIST_BYTES % 16 == 0, "chunk histograms as 16-byte words");
    constexpr int NW = static_cast<int>(HIST_BYTES / 16);
    // straight from global memory into LDS (global_load_lds_dwordx4: lane l
    // of a wave writes 16 bytes at the wave's LDS base + 16 l), no registers
    const uint4* src = reinterpret_cast<const uint4*>(x.hsplit + static_cast<size_t>(r) * NCH * CHW);
    constexpr int NK = (NW + NT - 1) / NT;
#pragma unroll
    for (int k = 0; k < NK; ++k) {
      const int i = k * NT + tid;
      if (i < NW)
        __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)(src + i),
                                         (__attribute__((address_space(3))) void*)(lds + 16 * (k * NT + (tid & ~63))), 16, 0, 0);
    }
    unsigned long long cr[NCH];
#pragma unroll
    for (int c = 0; c < NCH; ++c) cr[c] = x.crec[r * NCH + c];
    __builtin_amdgcn_s_waitcnt(0);
    // the largest bin over the chunks; the first chunk holding it has the
    // row's lowest index of it
    int cm = -65536;
#pragma unroll
    for (int c = 0; c < NCH; ++c) cm = max(cm, static_cast<int>(static_cast<unsigned>(cr[c])) - 65536);
    bmax = cm + NWIN + 1;
    fb = bmax == B_POSHUGE || bmax == B_TINY || bmax == B_NEGHUGE;
    if (!md.sampling) {
      id = INT_MAX;
#pragma unroll
      for (int c = NCH - 1; c >= 0; --c)
        if (static_cast<int>(static_cast<unsigned>(cr[c])) - 65536 == cm) id = static_cast<int>(cr[c] >> 32);
      fb = fb || id == INT_MAX;
    }
    __syncthreads();
    MLXF_RH_STAMP(1);
  } else {
    // ---- pass 1: every element counted once
    int best = -(NWIN + 1) - 1;  // (bin offset; below every bin)
    int bestit = -1;
    count_row<RH_DEPTH, PK>(lds, row, V, x.ipc, x.nfull, best, bestit);
    __syncthreads();
    MLXF_RH_STAMP(1);

    // ---- the row maximum (its bin); its lowest index only for greedy rows
    bmax = bmax_i(best, &sc.ir[0][0]) + NWIN + 1;
    fb = bmax == B_POSHUGE || bmax == B_TINY || bmax == B_NEGHUGE;
    if (!md.sampling) {
      const int myarg = best + NWIN + 1 == bmax && bestit >= 0 ? first_at(row, V, bestit, bmax) : INT_MAX;
      id = bmin_i(myarg, &sc.ir[0][0]);
      fb = fb || id == INT_MAX;
    }
  }
  const float M = bin_value(bmax);
  MLXF_RH_WSTAMP(0);

  // the thread's bins (descending from the top) and their counts
  int cnt[BPT];
#pragma unroll
  for (int j = 0; j < BPT; ++j) {
    const int b = own_bin(tid, j);
    cnt[j] = b >= 0 ? static_cast<int>(htot<PK>(hist, b)) : 0;
  }

  // ---- per-bin work, branch-free over the thread's bins: the log-sum-exp of
  // the unscaled row, and for a sampling row the weight of each bin (0 for an
  // empty one; a bin's fixed-point mass is q40 of it)
  const int wid = tid >> 6;
  const bool do_lse = md.need_lse && !fb;
  const bool do_w = md.sampling && !fb;
  float Mp = 0.0f, nc = 0.0f;
  if (do_w) {
    Mp = zdiv<DT>(M, md.Tr, md.y, false);
    nc = -(Mp * LOG2E);
  }
  // every window value is in the fast division's range (2^-96 <= |z| < 2^100)
  const bool fast = !md.tslow;
  // z' of a bin: -inf for the low bin (its mass is zero, checked below), 0
  // for the tiny bin (its elements' weights are equal, checked below)
  auto zp_of = [&](int b) -> float {
    if (b <= B_NEGHUGE || b >= B_POSHUGE) return -INFINITY;
    return b == B_TINY ? 0.0f : zdiv<DT>(bin_value(b), md.Tr, md.y, fast);
  };
  MLXF_RH_WSTAMP(1);
  // (the thread's 11 terms summed in fp32, relative error below 2^-20, then
  // the block sum in fp64)
  double part = 0.0;
  if (do_lse) {
    float pf = 0.0f;
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      const int b = own_bin(tid, j);
      const float e = static_cast<float>(cnt[j]) * wexp(bin_value(b), M);
      pf += (cnt[j] > 0 && b > B_NEGHUGE) ? e : 0.0f;
    }
    part = static_cast<double>(pf);
  }
  float w[BPT];
  unsigned long long q[BPT];
  if (do_w) {
#pragma unroll
    for (int j = 0; j < BPT; ++j) {
      const float z = cnt[j] > 0 ? zp_of(own_bin(tid, j)) : -INFINITY;
      w[j] = z == -INFINITY ? 0.0f : wfun(z, Mp, nc, false);
      q[j] = q40(w[j]);
    }
  }
  MLXF_RH_WSTAMP(2);
  // one barrier publishes the per-wave log-sum-exp partials and thread 0's
  // checks of the merged bins
  if (do_lse) {
    part = wave_sum(part);
    if (lane == 0) sc.dr[wid] = part;
  }
  if (do_w && tid == 0) {
    bool bad = !__builtin_isfinite(Mp);
    if (!bad && htot<PK>(hist, B_TINY) > 0u) {
      // |z'| of a tiny value is below 2^-28 / T (rounded up by the bf16
      // rounding); the weight's log2 offset nc must absorb it
      const float zb = 0x1p-28f / md.Tr * 1.0078125f;
      const int e = nc == 0.0f ? -1000 : ilogbf(nc);
      bad = !(zb * LOG2E * 1.0001f < ldexpf(1.0f, e - 24));
    }
    if (!bad && htot<PK>(hist, B_NEGHUGE) > 0u) {
      // the largest value of the low bin, -256, must carry no mass
      bad = q40(wfun(zdiv<DT>(-256.0f, md.Tr, md.y, false), Mp, nc, false)) != 0ull;
    }
    sc.sel[0] = bad ? 1 : 0;
    sc.sel[3] = -1;
    sc.sel[4] = -1;
    sc.sel[5] = 0;
    sc.sel[6] = INT_MAX;
  }
  MLXF_RH_WSTAMP(3);
  __syncthreads();
  MLXF_RH_WSTAMP(4);
  double lse = static_cast<double>(NAN);
  if (do_lse) lse = static_cast<double>(M) + log(rdl(row_sum16(lane < NWV ? sc.dr[lane & (NWV - 1)] : 0.0), 0));
  MLXF_RH_STAMP(2);

  if (do_w) {
    fb = sc.sel[0] != 0;
    MLXF_RH_STAMP(3);

    // The tie group of bin bb: the run of adjacent bins with z' == z'(bb) (z'
    // is monotone in z), found by one wave 64 bins per step.  A group at or
    // next to a merged bin cannot be ordered exactly (the fallback).
    auto group_of = [&](int bb, int* glo, int* ghi) {
      const float zb = zp_of(bb);
      int lo = bb, hi = bb;
      for (;;) {
        const int b = lo - 1 - lane;
        const unsigned long long m = __ballot(b >= 0 && zp_of(b) == zb);
        const int run = m == ~0ull ? 64 : __ffsll(static_cast<long long>(~m)) - 1;
        lo -= run;
        if (run < 64) break;
      }
      for (;;) {
        const int b = hi + 1 + lane;
        const unsigned long long m = __ballot(b < NBIN && zp_of(b) == zb);
        const int run = m == ~0ull ? 64 : __ffsll(static_cast<long long>(~m)) - 1;
        hi += run;
        if (run < 64) break;
      }
      *glo = lo;
      *ghi = hi;
    };
    auto near_merged = [](int glo, int ghi) {
      return glo <= B_NEGHUGE + 1 || (glo <= B_TINY + 1 && ghi >= B_TINY - 1) || ghi >= B_POSHUGE - 1;
    };
    // (whole wave) count of row elements in bins [lo, hi], from the histograms
    auto count_range = [&](int lo, int hi) -> int {
      int c = 0;
      for (int b = lo + lane; b <= hi; b += 64)
        c += static_cast<int>(htot<PK>(hist, b));
      return wave_sum(c);
    };
    // (wave 0, whole wave) the chunk holding the draw, from lane c < NSUB's
    // chunk c kept mass K, partial-group elements G and kept-bin elements N:
    // sel[1] = the chunk, sel[2] = its kept ties, sel[14] = its elements at
    // or above the cutoff, sel64[0] = the draw's offset into its kept mass
    auto chunk_pick = [&](unsigned long long K, int G, int N, const Kept& k) {
      // the first t ties in index order are spread over the chunks in order
      const int before = wave_incl_scan_dpp(G) - G;
      const unsigned int want = k.t > static_cast<unsigned>(before) ? k.t - static_cast<unsigned>(before) : 0u;
      const unsigned int tk = want < static_cast<unsigned>(G) ? want : static_cast<unsigned>(G);
      K += static_cast<unsigned long long>(tk) * k.wt;
      const unsigned long long cumi = wave_incl_scan_dpp(K);
      const unsigned long long W = rdl(cumi, 63);
      unsigned long long Tu = static_cast<unsigned long long>(static_cast<double>(md.u) * static_cast<double>(W));
      if (W == 0ull)
        Tu = 0ull;
      else if (Tu >= W)
        Tu = W - 1ull;
      const unsigned long long hit = __ballot(lane < NSUB && K > 0ull && cumi > Tu);
      const int cs = hit ? __ffsll(static_cast<long long>(hit)) - 1 : -1;
      // (lane reads with the whole wave active: a value computed only in
      // the lane-0 branch would not exist in lane cs)
      const int csr = cs >= 0 ? cs : 0;
      const int tks = static_cast<int>(rdl(tk, csr));
      const int ngs = rdl(N + G, csr);
      const unsigned long long rems = Tu - (rdl(cumi, csr) - rdl(K, csr));
      if (lane == 0) {
        sc.sel[1] = cs;
        sc.sel[2] = cs >= 0 ? tks : 0;
        sc.sel[14] = cs >= 0 ? ngs : 0;
        sc.sel64[0] = cs >= 0 ? rems : 0ull;
      }
    };
    // (wave 0, whole wave) chunk_pick for a kept range [need, bmax] of at most
    // 4 x 64 bins, lane i taking bins bmax - i - 64 j (weights recomputed, a
    // bin with no elements skipped): no other wave takes part.  False (nothing
    // done) for a wider range.
    auto narrow_chunks = [&](const Kept& k) -> bool {
      const int need = k.t > 0u ? k.glo : k.kb;
      const int nr = (bmax - need + 64) >> 6;  // rounds of 64 bins
      if (nr > 4) return false;
      // per chunk: kept mass, and (packed) kept-bin elements << 32 | partial-group elements
      unsigned long long kc[NSUB], gn[NSUB];
#pragma unroll
      for (int c = 0; c < NSUB; ++c) {
        kc[c] = 0ull;
        gn[c] = 0ull;
      }
      for (int j = 0; j < nr; ++j) {
        const int b = bmax - lane - 64 * j;
        const bool in = b >= need;
        unsigned int h[NSUB];
        unsigned int any = 0u;
#pragma unroll
        for (int c = 0; c < NSUB; ++c) {
          h[c] = in ? hsub<PK>(hist, c, b) : 0u;
          any |= h[c];
        }
        if (any != 0u) {
          if (b >= k.kb) {
            const unsigned long long qq = q40(wfun(zp_of(b), Mp, nc, false));
#pragma unroll
            for (int c = 0; c < NSUB; ++c) {
              kc[c] += static_cast<unsigned long long>(h[c]) * qq;
              gn[c] += static_cast<unsigned long long>(h[c]) << 32;
            }
          } else {
#pragma unroll
            for (int c = 0; c < NSUB; ++c) gn[c] += h[c];
          }
        }
      }
      // lane c < NSUB: chunk c's sums (held by lane c * 64 / NSUB after the
      // reduce-scatter)
      const unsigned long long kcs = wave_rs<NSUB>(kc), gns = wave_rs<NSUB>(gn);
      const int src = (lane < NSUB ? lane : 0) * (64 / NSUB);
      const unsigned long long K0 = shfl_u64(kcs, src), GN0 = shfl_u64(gns, src);
      const unsigned long long K = lane < NSUB ? K0 : 0ull, GN = lane < NSUB ? GN0 : 0ull;
      const int G = static_cast<int>(static_cast<unsigned int>(GN)), N = static_cast<int>(GN >> 32);
      chunk_pick(K, G, N, k);
      return true;
    };

    // the kept set so far, as published by wave 0 in sc: kb (sel[10]), the
    // partial group glo, ghi, t (sel[11..13]) and its mass (sel64[3])
    Kept kp;
    kp.kb = 0;
    kp.glo = 0;
    kp.ghi = -1;
    kp.t = 0u;
    kp.wt = 0ull;
    // top-k: the k'-th largest z' counting multiplicity; its ties are kept
    if (!fb && md.kk > 0) {
      int csum = 0;
#pragma unroll
      for (int j = 0; j < BPT; ++j) csum += cnt[j];
      int ctot;
      const int run = bscan(csum, &sc.ir[0][0], &ctot);
      if (run < md.kk && md.kk <= run + csum) {  // the one thread holding the k'-th
        int rr = run;
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
          if (cnt[j] > 0 && rr < md.kk && rr + cnt[j] >= md.kk) sc.sel[3] = own_bin(tid, j);
          rr += cnt[j];
        }
      }
      __syncthreads();
      if (wid == 0) {
        const int bk = sc.sel[3];
        int glo = 0, ghi = 0;
        if (bk >= 0) group_of(bk, &glo, &ghi);
        const bool bad = bk < 0 || near_merged(glo, ghi);
        bool done = false;
        if (!bad && !(md.topp || md.mr > 0.0f)) {
          // the kept set is final: every bin >= glo
          Kept k2;
          k2.kb = glo;
          k2.glo = 0;
          k2.ghi = -1;
          k2.t = 0u;
          k2.wt = 0ull;
          done = narrow_chunks(k2);
        }
        if (lane == 0) {
          sc.sel[10] = glo;
          sc.sel[0] = bad ? 1 : 0;
          sc.sel[5] = done ? 1 : 0;
        }
      }
      __syncthreads();
      kp.kb = sc.sel[10];
      fb = sc.sel[0] != 0;
    }
    const int klo = kp.kb;
    MLXF_RH_STAMP(4);
    // top-p over the top-k survivors (keep while the mass before an element,
    // in z' desc / index asc order, is below ceil(p * W)), and min_p after it
    // (the weights that reach min_p times the max's; the lowest such occupied
    // bin, empty bins below it changing nothing); both from one pass over the
    // bins
    if (!fb && (md.topp || md.mr > 0.0f)) {
      MLXF_RH_STAMP(11);
      const float thr = md.mr > 0.0f ? minp_thr(md.mr, Mp, nc, false) : 0.0f;
      if (md.mr > 0.0f) {
        int lo = INT_MAX;
#pragma unroll
        for (int j = 0; j < BPT; ++j)
          if (w[j] >= thr && cnt[j] > 0) lo = min(lo, own_bin(tid, j));
        lo = wave_min(lo);
        if (lane == 0 && lo != INT_MAX) atomicMin(&sc.sel[6], lo);
      }
      unsigned long long PW = 0ull;
      if (md.topp) {
        auto mass = [&](int j) -> unsigned long long {
          return own_bin(tid, j) >= klo ? static_cast<unsigned long long>(cnt[j]) * q[j] : 0ull;
        };
        unsigned long long msum = 0ull;
#pragma unroll
        for (int j = 0; j < BPT; ++j)
          if (cnt[j] > 0) msum += mass(j);
        unsigned long long Wk;
        const unsigned long long run = bscan(msum, &sc.u64r[0][0], &Wk);
        PW = static_cast<unsigned long long>(ceil(static_cast<double>(md.pr) * static_cast<double>(Wk)));
        if (PW < 1ull) PW = 1ull;
        if (run < PW && PW <= run + msum) {  // the one thread holding the cutoff
          unsigned long long rr = run;
#pragma unroll
          for (int j = 0; j < BPT; ++j) {
            const unsigned long long mj = mass(j);
            if (mj > 0ull && rr < PW && rr + mj >= PW) {
              sc.sel[4] = own_bin(tid, j);
              sc.sel64[2] = rr;  // mass of the bins above it
            }
            rr += mj;
          }
        }
      }
      __syncthreads();
      MLXF_RH_STAMP(12);
      if (wid == 0) {
        int kb = klo, glo = 0, ghi = -1;
        unsigned int t = 0u;
        unsigned long long wt = 0ull;
        bool bad = false;
        if (md.topp) {
          const int bp = sc.sel[4];
          if (bp >= 0) group_of(bp, &glo, &ghi);
          bad = bp < 0 || near_merged(glo, ghi);
          if (!bad) {
            // the group's bins share one weight: its elements, and the mass
            // above the group = the mass above bp less the group's bins above bp
            wt = q40(wfun(zp_of(bp), Mp, nc, false));
            const unsigned int gcnt = static_cast<unsigned int>(count_range(glo, ghi));
            const unsigned long long above =
                sc.sel64[2] - static_cast<unsigned long long>(count_range(bp + 1, ghi)) * wt;
            t = ties_kept(PW > above ? PW - above : 0ull, wt, gcnt);
            if (t >= gcnt) {
              kb = glo;  // the whole group is kept
              t = 0u;
            } else {
              kb = ghi + 1;
            }
          }
        }
        if (!bad && md.mr > 0.0f) {
          const int bm = sc.sel[6];
          const int low_kept = t > 0u ? glo : kb;  // lowest bin with a kept element
          if (bm > low_kept) {
            kb = max(kb, bm);
            t = 0u;
          }
        }
        bool done = false;
        if (!bad) {
          Kept k2;
          k2.kb = kb;
          k2.glo = t > 0u ? glo : 0;
          k2.ghi = t > 0u ? ghi : -1;
          k2.t = t;
          k2.wt = t > 0u ? wt : 0ull;
          done = narrow_chunks(k2);
        }
        if (lane == 0) {
          sc.sel[0] = bad ? 1 : 0;
          sc.sel[5] = done ? 1 : 0;
          sc.sel[10] = kb;
          sc.sel[11] = glo;
          sc.sel[12] = ghi;
          sc.sel[13] = static_cast<int>(t);
          sc.sel64[3] = wt;
        }
      }
      MLXF_RH_STAMP(13);
      __syncthreads();
      fb = sc.sel[0] != 0;
      kp.kb = sc.sel[10];
      kp.t = static_cast<unsigned int>(sc.sel[13]);
      if (kp.t > 0u) {
        kp.glo = sc.sel[11];
        kp.ghi = sc.sel[12];
        kp.wt = sc.sel64[3];
      }
    }
    MLXF_RH_STAMP(5);
    MLXF_RH_STAMP(6);

    if (!fb) {
      // ---- per-chunk kept masses and the chunk holding u * W
      const int need_lo = kp.t > 0u ? kp.glo : kp.kb;
      // per chunk: kept mass kc, partial-group elements gc, and elements of
      // the wholly kept bins nk (unless wave 0 has picked the chunk already)
      MLXF_RH_WSTAMP(12);
      if (sc.sel[5] == 0) {
        // Per chunk, over the thread's own bins: kept mass kc (as h * low 32
        // bits of the mass in 64 bits plus h * high bits in 32: h < 2^16 and
        // a mass < 2^41), kept-bin elements nk and partial-group elements gc.
        // A wave whose highest bin is below every kept one adds nothing.
        unsigned long long kcs = 0ull, gns = 0ull;
        if (own_bin(wid * 64, 0) >= need_lo) {
          unsigned long long kl[NSUB];
          unsigned int kh[NSUB], nk[NSUB], gc[NSUB];
#pragma unroll
          for (int c = 0; c < NSUB; ++c) {
            kl[c] = 0ull;
            kh[c] = 0u;
            nk[c] = 0u;
            gc[c] = 0u;
          }
          if (own_bin(tid, 0) >= need_lo) {
#pragma unroll
            for (int j = 0; j < BPT; ++j) {
              const int b = own_bin(tid, j);
              if (b < 0 || cnt[j] == 0) continue;
              if (b >= kp.kb) {
                const unsigned int qlo = static_cast<unsigned int>(q[j]), qhi = static_cast<unsigned int>(q[j] >> 32);
#pragma unroll
                for (int c = 0; c < NSUB; ++c) {
                  const unsigned int h = hsub<PK>(hist, c, b);
                  kl[c] += static_cast<unsigned long long>(h) * qlo;
                  kh[c] += h * qhi;
                  nk[c] += h;
                }
              } else if (kp.t > 0u && b >= kp.glo && b <= kp.ghi) {
#pragma unroll
                for (int c = 0; c < NSUB; ++c) gc[c] += hsub<PK>(hist, c, b);
              }
            }
          }
          unsigned long long kc[NSUB], gn[NSUB];
#pragma unroll
          for (int c = 0; c < NSUB; ++c) {
            kc[c] = kl[c] + (static_cast<unsigned long long>(kh[c]) << 32);
            gn[c] = (static_cast<unsigned long long>(nk[c]) << 32) | gc[c];
          }
          // the wave's sums of chunk c in lanes c * 64 / NSUB ...
          kcs = wave_rs<NSUB>(kc);
          gns = wave_rs<NSUB>(gn);
        }
        MLXF_RH_WSTAMP(8);
        if ((lane & (64 / NSUB - 1)) == 0) {
          sc.u64r[wid][lane / (64 / NSUB)] = kcs;
          sc.ugn[wid][lane / (64 / NSUB)] = gns;
        }
        __syncthreads();
        MLXF_RH_WSTAMP(9);
        if (wid == 0) {
          // ... and lane c < NSUB's over the waves
          unsigned long long K = 0ull, GN = 0ull;
          if (lane < NSUB) {
#pragma unroll
            for (int w2 = 0; w2 < NWV; ++w2) {
              K += sc.u64r[w2][lane];
              GN += sc.ugn[w2][lane];
            }
          }
          MLXF_RH_WSTAMP(10);
          chunk_pick(K, static_cast<int>(static_cast<unsigned int>(GN)), static_cast<int>(GN >> 32), kp);
          MLXF_RH_WSTAMP(11);
        }
      }
      __syncthreads();
      const int cs = sc.sel[1];
      const unsigned int tkc = static_cast<unsigned int>(sc.sel[2]);
      const unsigned long long rem = sc.sel64[0];
      fb = cs < 0;
      MLXF_RH_STAMP(7);
      if (!fb) {
        // the walk's chunk: ips iterations' elements, EPTW consecutive ones
        // per thread
        const int ips = PK ? x.ipc >> 1 : x.ipc;
        const int EPTW = ips * 8;
        const int c0 = cs * ips * ITER + tid * EPTW;
        // the thread's first 16-byte words of the walk requested before the
        // weight table is built (the table needs the histograms to be dead)
        constexpr int WG = 8;
        uint4 wq[WG];
        const bool whole = c0 + EPTW <= V;
        if (whole) {
          const uint4* rv = reinterpret_cast<const uint4*>(row + c0);
#pragma unroll
          for (int k = 0; k < WG; ++k)
            if (k < EPTW / 8) wq[k] = rv[k];
        }
        MLXF_RH_WSTAMP(13);
        if (sc.sel[14] <= SPARSE && EPTW <= 64) {
          // ---- sparse draw: the chunk's few elements at or above need_lo,
          // listed in index order (each thread's qualifying elements at its
          // exclusive-scan offset), then walked by wave 0
          unsigned long long mk = 0ull;  // bit e: element c0 + e qualifies
          if (whole) {
#pragma unroll
            for (int k = 0; k < WG; ++k) {
              if (k < EPTW / 8) {
                const unsigned int w4[4] = {wq[k].x, wq[k].y, wq[k].z, wq[k].w};
#pragma unroll
                for (int h = 0; h < 4; ++h) {
                  const unsigned int b2 = bins2(w4[h]);
                  mk |= static_cast<unsigned long long>(static_cast<int>(b2 & 0xffffu) >= need_lo) << (8 * k + 2 * h);
                  mk |= static_cast<unsigned long long>(static_cast<int>(b2 >> 16) >= need_lo) << (8 * k + 2 * h + 1);
                }
              }
            }
          } else {
            for (int e = 0; e < EPTW; ++e) {
              const int p = c0 + e;
              if (p < V && static_cast<int>(bins2(row[p]) & 0xffffu) >= need_lo) mk |= 1ull << e;
            }
          }
          int ntot;
          int o = bscan(static_cast<int>(__builtin_popcountll(mk)), &sc.ir[0][0], &ntot);
          while (mk) {
            const int e = __ffsll(static_cast<long long>(mk)) - 1;
            mk &= mk - 1ull;
            if (o < SPARSE) sc.lst[o] = static_cast<unsigned int>(c0 + e);
            ++o;
          }
          __syncthreads();
          if (wid == 0) {
            // (ntot equals the histograms' count; the guard only keeps the
            // list reads in bounds)
            const int n = min(ntot, SPARSE);
            unsigned long long carry = 0ull;
            unsigned int tie_rank = 0u;
            int found = -1;
            for (int i0 = 0; i0 < n && found < 0; i0 += 64) {
              const bool valid = i0 + lane < n;
              const int p = valid ? static_cast<int>(sc.lst[i0 + lane]) : 0;
              const int b = valid ? static_cast<int>(bins2(row[p]) & 0xffffu) : B_TRASH;
              unsigned long long mm = 0ull;
              if (valid && b >= kp.kb) mm = q40(wfun(zp_of(b), Mp, nc, false));
              if (kp.t > 0u) {
                const bool tie = valid && b >= kp.glo && b <= kp.ghi;
                const unsigned long long tb = __ballot(tie);
                const unsigned int rk = tie_rank + __builtin_amdgcn_mbcnt_hi(static_cast<unsigned int>(tb >> 32),
                                                                            __builtin_amdgcn_mbcnt_lo(static_cast<unsigned int>(tb), 0u));
                if (tie && rk < tkc) mm = kp.wt;
                tie_rank += static_cast<unsigned int>(__builtin_popcountll(tb));
              }
              const unsigned long long c = carry + wave_incl_scan_dpp(mm);
              const int pk = wave_min((mm > 0ull && c > rem) ? p : INT_MAX);
              if (pk != INT_MAX) found = pk;
              carry = rdl(c, 63);
            }
            if (lane == 0) sc.sel[9] = ntot == sc.sel[14] ? found : -1;
          }
          __syncthreads();
          id = sc.sel[9];
          fb = id < 0;
        } else {
        // the weight table over the dead histograms: each wholly kept bin's
        // mass at byte 8 * bin, 0 for every other bin
        unsigned long long* tab = reinterpret_cast<unsigned long long*>(lds);
        __syncthreads();
        MLXF_RH_WSTAMP(14);
#pragma unroll
        for (int j = 0; j < BPT; ++j) {
          const int b = own_bin(tid, j);
          if (b >= 0) tab[b] = (b >= kp.kb && cnt[j] > 0) ? q[j] : 0ull;
        }
        if (tid == 0) tab[B_TRASH] = 0ull;
        MLXF_RH_WSTAMP(15);
        __syncthreads();
        MLXF_RH_WSTAMP(5);
        const unsigned long long km0 = kp.t > 0u ? walk_sum<true, WG>(row, V, c0, EPTW, tab, kp, wq, whole)
                                                 : walk_sum<false, WG>(row, V, c0, EPTW, tab, kp, wq, whole);
        unsigned long long km = km0 & 0x00ffffffffffffffull;  // (mass; tie count in the top byte, see walk_sum)
        const int gt = static_cast<int>(km0 >> 56);
        MLXF_RH_WSTAMP(6);
        MLXF_RH_STAMP(8);
        // one scan of the wholly kept mass and the partial group's elements;
        // the first tkc of those (index order) are kept, so the threads before
        // this one keep min(gex, tkc) of them
        if (tid == 0) sc.sel[7] = -1;
        unsigned long long kex, ktot;
        int gex, gtot;
        bscan2(km, gt, &sc.u64r[0][0], &sc.ir[0][0], &kex, &gex, &ktot, &gtot);
        if (kp.t > 0u) {
          const unsigned int kt = tkc > static_cast<unsigned>(gex)
                                      ? min(tkc - static_cast<unsigned>(gex), static_cast<unsigned>(gt))
                                      : 0u;
          km += static_cast<unsigned long long>(kt) * kp.wt;
          kex += static_cast<unsigned long long>(min(static_cast<unsigned>(gex), tkc)) * kp.wt;
        }
        if (km > 0ull && kex <= rem && rem < kex + km) {
          sc.sel[7] = tid;
          sc.sel[8] = gex;
          sc.sel64[1] = rem - kex;
        }
        __syncthreads();
        MLXF_RH_WSTAMP(7);
        MLXF_RH_STAMP(9);
        const int holder = sc.sel[7];
        if (holder >= 0 && tid < 64) {
          // wave 0 walks the holder's elements, one per lane per round
          const int hbase = cs * ips * ITER + holder * EPTW;
          const unsigned long long hrem = sc.sel64[1];
          unsigned int tie_rank = static_cast<unsigned int>(sc.sel[8]);
          unsigned long long carry = 0ull;
          int found = -1;
          for (int e0 = 0; e0 < EPTW && found < 0; e0 += 64) {
            const int p = hbase + e0 + lane;
            const bool valid = e0 + lane < EPTW && p < V;
            const unsigned int bits = valid ? row[p] : 0u;
            const int b = valid ? static_cast<int>(bins2(bits) & 0xffffu) : B_TRASH;
            unsigned long long mm = tab[b];
            if (kp.t > 0u) {
              const bool tie = valid && b >= kp.glo && b <= kp.ghi;
              const unsigned long long tb = __ballot(tie);
              const unsigned int rk = tie_rank + __builtin_amdgcn_mbcnt_hi(static_cast<unsigned int>(tb >> 32),
                                                                          __builtin_amdgcn_mbcnt_lo(static_cast<unsigned int>(tb), 0u));
              if (tie && rk < tkc) mm = kp.wt;
              tie_rank += static_cast<unsigned int>(__builtin_popcountll(tb));
            }
            const unsigned long long c = carry + wave_incl_scan_dpp(mm);
            const int pk = wave_min((mm > 0ull && c > hrem) ? p : INT_MAX);
            if (pk != INT_MAX) found = pk;
            carry = rdl(c, 63);
          }
          if (lane == 0) sc.sel[9] = found;
        }
        __syncthreads();
        id = holder >= 0 ? sc.sel[9] : -1;
        fb = id < 0;
        }
      }
    }
  }
  MLXF_RH_STAMP(10);
  if (!fb) {
    if (tid == 0) write_out<DT>(a, r, id, lse, md.want_lp);
    return;
  }
  // ---- the fallback (fb is the same in every thread): the per-slice path
  // over this row in waves 0..3, on the LDS the histograms leave.  The other
  // waves end here; a barrier waits for the waves that have not ended.
  __syncthreads();
  if (tid >= THREADS) return;
  // (a is the kernel's first argument: offset 0 of the argument segment)
  row_fallback<DT, EPT>((__attribute__((address_space(4))) const Args*)__builtin_amdgcn_kernarg_segment_ptr(), r,
                        (__attribute__((address_space(3))) unsigned char*)lds);
}

// One call on the row-histogram path: k_row16 over every row; with few rows
// (x.hsplit set) the chunks are first counted in parallel by k_cnt16.
template <int DT, int EPT>
hipError_t launch_row16(const Args& a, const RhArgs& x, hipStream_t st) {
  static_assert(sizeof(FbShared) <= rh::LDS_BYTES, "the fallback's LDS must fit in the histograms'");
  if (x.hsplit) {
    const unsigned int groups = static_cast<unsigned int>((a.B + 7) / 8);
    hipLaunchKernelGGL((k_cnt16<DT>), dim3(groups * 8u * rh::NCH), dim3(rh::NT), 0, st, a, x);
    hipLaunchKernelGGL((k_row16<DT, EPT, true>), dim3(static_cast<unsigned int>(a.B)), dim3(rh::NT), 0, st, a, x);
  } else {
    hipLaunchKernelGGL((k_row16<DT, EPT, false>), dim3(static_cast<unsigned int>(a.B)), dim3(rh::NT), 0, st, a, x);
  }
  return hipGetLastError();
}

template <int DT>
hipError_t launch_row16_dt(const Args& a, int ept, const RhArgs& x, hipStream_t st) {
  switch (ept) {
    case 8:
      return launch_row16<DT, 8>(a, x, st);
    case 16:
      return launch_row16<DT, 16>(a, x, st);
    default:
      return launch_row16<DT, 32>(a, x, st);
  }
}

}  // namespace
}  // namespace mlxf
