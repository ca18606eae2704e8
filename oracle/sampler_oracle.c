/*
 * sampler_oracle.c -- CPU restatement of mlxforge's batched token sampler.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the GPU path is compared
 * against (parity tests under tests/, __graft_entry__.smoke(), and bench.py's
 * cpu_baseline leg).  The product path (mlxforge_amd/) never links, loads or
 * calls it.
 *
 * It restates, per row and in plain C with fp64 accumulation, what the
 * reference computes with MLX graph ops:
 *   Sampler::sample   src/sample/sampler.cpp:141-166
 *   Sampler::greedy   src/sample/sampler.cpp:59-61
 *   apply_top_k       src/sample/sampler.cpp:63-68   (clamp k to V: :159-161)
 *   apply_top_p       src/sample/sampler.cpp:70-85
 *   apply_min_p       src/sample/sampler.cpp:87-93
 *   penalties         src/sample/sampler.cpp:95-133
 *   log_probs / gather_logprob / top_k_logprobs   src/sample/sampler.cpp:15-38
 *   per-row application in the decode step        src/runtime/worker.cpp:448-486
 *   parameter sanitisation                        src/capi/mlxforge.cpp:43-70
 *
 * The cost structure deliberately mirrors the reference (a full argsort of the
 * vocabulary for top-p and for top_logprobs, a quickselect for top-k, a full
 * softmax and a sequential cumulative sum) so that timing it gives a fair
 * "reference-shaped" CPU baseline.
 *
 * Decisions the reference leaves to MLX (which cannot run here) and which the
 * HIP kernels implement identically:
 *   D1  temperature is rounded to the logits dtype and z' = round_dtype(z / T)
 *       with IEEE fp32 division (sampler.cpp:158 divides by an array of T in the
 *       logits dtype).
 *   D2  sort order for top-p is (z' desc, index asc).
 *   D3  the nucleus mass is accumulated in fp64 here (fp32/fp64 on the GPU), not
 *       in the logits dtype.
 *   D4  the categorical draw is an inverse CDF in ascending vocabulary order with
 *       one caller-supplied uniform u per row:
 *         id = min{ j kept : sum_{i<=j, i kept} w_i > u * sum_kept w },
 *       w_i = exp(z'_i - max z').
 *   D5  logprobs are returned as fp32 for every input dtype.
 *   D6  for bf16/f16 logits p is rounded to the logits dtype
 *       (sampler.cpp:79 compares against array(p, probs.dtype())).
 *   D7  NaN logits are read as -inf; exp(x - max) is taken as 1 where x == max
 *       (so rows with +inf entries stay finite and well defined: their mass is
 *       split evenly over the +inf entries).  A row with nothing left to draw
 *       (all -inf, or a top-p that rounds to 0) returns index 0, the argmax of
 *       an all -inf row that MLX's Gumbel-max categorical takes.
 *   D8  top_logprobs alternatives are ordered by (z desc, index asc), the exact
 *       order of log_softmax(z).
 *   D9  min_p in (0, 1] (else off, src/capi/mlxforge.cpp:58) is rounded to the
 *       logits dtype like p (sampler.cpp:91 multiplies by array(min_p,
 *       probs.dtype())) and applied after top-p: keep exp(z' - max z') >= min_p.
 *   D10 a history id's count for the frequency penalty is its exact number of
 *       occurrences rounded once to the logits dtype (sampler.cpp:113 sums
 *       ones in the logits dtype; below 257 every order of summation agrees).
 *
 * Ambiguity flags (the north-star exclusion rule): a row whose top-p cutoff or
 * draw boundary lies within 1e-6 of the compared quantity is reported with
 * ORC_FLAG_TOPP_AMBIG / ORC_FLAG_DRAW_AMBIG; a weight other than the max's
 * within 1e-6 (relative) of min_p is ORC_FLAG_MINP_AMBIG.  Such a row is not
 * compared bit-exactly; orc_admissible() gives every id the row can produce
 * when p, u and min_p each move by up to 1e-6, and the GPU's id must be one
 * of them.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_F32 0
#define ORC_BF16 1
#define ORC_F16 2

#define ORC_FLAG_GREEDY 1
#define ORC_FLAG_TOPP_AMBIG 2
#define ORC_FLAG_DRAW_AMBIG 4
#define ORC_FLAG_MINP_AMBIG 8

#define ORC_AMBIG_EPS 1e-6

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* ---- dtype rounding (round-to-nearest-even) ------------------------------ */

float orc_round_bf16(float x) {
  uint32_t u = f2u(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return u2f((u | 0x00400000u) & 0xffff0000u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return u2f(u & 0xffff0000u);
}

uint16_t orc_f32_to_f16_bits(float f) {
  uint32_t x = f2u(f);
  uint32_t sign = (x >> 16) & 0x8000u;
  uint32_t ax = x & 0x7fffffffu;
  if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
  if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u); /* rounds to inf */
  if (ax < 0x38800000u) {                                   /* half subnormal */
    float v = u2f(ax) * 16777216.0f;                         /* exact: 2^24 */
    return (uint16_t)(sign | (uint32_t)nearbyintf(v));
  }
  uint32_t e = (ax >> 23) - 127u + 15u;
  uint32_t mant = ax & 0x7fffffu;
  uint32_t h = (e << 10) | (mant >> 13);
  uint32_t rem = mant & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
  return (uint16_t)(sign | h);
}

float orc_f16_bits_to_f32(uint16_t h) {
  uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
  uint32_t e = (h >> 10) & 0x1fu;
  uint32_t m = h & 0x3ffu;
  if (e == 0x1fu) return u2f(sign | 0x7f800000u | (m << 13));
  if (e == 0) {
    float v = (float)m * (1.0f / 16777216.0f);
    return sign ? -v : v;
  }
  return u2f(sign | ((e - 15u + 127u) << 23) | (m << 13));
}

float orc_round_f16(float x) { return orc_f16_bits_to_f32(orc_f32_to_f16_bits(x)); }

static inline float round_dtype(float x, int dtype) {
  if (dtype == ORC_BF16) return orc_round_bf16(x);
  if (dtype == ORC_F16) return orc_round_f16(x);
  return x;
}

/* Element read; NaN is read as -inf (D7). */
static inline float load_logit(const void* base, int dtype, size_t i) {
  float v;
  if (dtype == ORC_BF16)
    v = u2f((uint32_t)((const uint16_t*)base)[i] << 16);
  else if (dtype == ORC_F16)
    v = orc_f16_bits_to_f32(((const uint16_t*)base)[i]);
  else
    v = ((const float*)base)[i];
  return isnan(v) ? -INFINITY : v;
}

/* exp(x - m) with the D7 convention exp(m - m) = 1 even for infinite m. */
static inline double wexp(float x, float m) { return x == m ? 1.0 : exp((double)x - (double)m); }

/* ---- orderings ------------------------------------------------------------ */

typedef struct {
  float v;
  int32_t i;
} vi_t;

/* (value desc, index asc) -- D2 / D8 */
static int cmp_desc_idx(const void* a, const void* b) {
  const vi_t* x = (const vi_t*)a;
  const vi_t* y = (const vi_t*)b;
  if (x->v > y->v) return -1;
  if (x->v < y->v) return 1;
  return (x->i > y->i) - (x->i < y->i);
}

/* k-th largest (1-based) of a[0..n) counting multiplicity; a is permuted.
 * Hoare-style quickselect (the std::nth_element shape that mx::topk stands for,
 * src/sample/sampler.cpp:65). */
static float kth_largest(float* a, int n, int k) {
  int lo = 0, hi = n - 1, target = k - 1; /* index in descending order */
  while (lo < hi) {
    float pivot = a[lo + (hi - lo) / 2];
    int i = lo, j = hi;
    while (i <= j) {
      while (a[i] > pivot) i++;
      while (a[j] < pivot) j--;
      if (i <= j) {
        float t = a[i];
        a[i] = a[j];
        a[j] = t;
        i++;
        j--;
      }
    }
    if (target <= j)
      hi = j;
    else if (target >= i)
      lo = i;
    else
      break;
  }
  return a[target];
}

/* ---- the reference's building blocks, on one row ------------------------- */

/* argmax, lowest index on ties (src/sample/sampler.cpp:59-61). */
int orc_greedy_row(const float* z, int V) {
  int best = 0;
  for (int i = 1; i < V; ++i)
    if (z[i] > z[best]) best = i;
  return best;
}

/* log-sum-exp of the unscaled row (src/sample/sampler.cpp:15-17, softmax precise). */
double orc_lse_row(const float* z, int V) {
  float m = z[0];
  for (int i = 1; i < V; ++i)
    if (z[i] > m) m = z[i];
  double s = 0.0;
  for (int i = 0; i < V; ++i) s += wexp(z[i], m);
  return (double)m + log(s);
}

/* In place: z'_i < tau_k -> -inf, tau_k = k-th largest (ties at tau_k kept).
 * src/sample/sampler.cpp:63-68; k clamped to V as at :159-161. */
void orc_apply_top_k(float* zs, int V, int k) {
  if (k <= 0) return;
  if (k > V) k = V;
  float* tmp = (float*)malloc(sizeof(float) * (size_t)V);
  memcpy(tmp, zs, sizeof(float) * (size_t)V);
  float tau = kth_largest(tmp, V, k);
  free(tmp);
  for (int i = 0; i < V; ++i)
    if (zs[i] < tau) zs[i] = -INFINITY;
}

/* In place: keep the smallest (z' desc, index asc) prefix whose prior mass is
 * < p (src/sample/sampler.cpp:70-85).  `pc` is p already cast to the probs
 * dtype.  Returns ambiguity flags; *margin gets min distance of the cutoff's
 * prior masses to p. */
int orc_apply_top_p(float* zs, int V, float pc, double* margin) {
  vi_t* ord = (vi_t*)malloc(sizeof(vi_t) * (size_t)V);
  for (int i = 0; i < V; ++i) {
    ord[i].v = zs[i];
    ord[i].i = i;
  }
  qsort(ord, (size_t)V, sizeof(vi_t), cmp_desc_idx); /* argsort(-z'), :72 */
  const float m = ord[0].v;
  double W = 0.0;
  for (int j = 0; j < V; ++j) W += wexp(ord[j].v, m); /* softmax denom, :74 */
  const double pW = (double)pc * W;
  double prior = 0.0;
  double mg = INFINITY;
  int last_kept = -1;
  for (int j = 0; j < V; ++j) {
    const double q = wexp(ord[j].v, m);
    const int keep = prior < pW; /* :78-79, keep iff prior mass < p */
    if (!keep) {
      if (j == last_kept + 1) {
        double d = prior / W - (double)pc;
        if (fabs(d) < mg) mg = fabs(d);
      }
      zs[ord[j].i] = -INFINITY; /* :80-84 */
    } else {
      last_kept = j;
    }
    prior += q;
  }
  /* margin of the last kept element */
  if (last_kept >= 0) {
    double pr = 0.0;
    for (int j = 0; j < last_kept; ++j) pr += wexp(ord[j].v, m);
    double d = (double)pc - pr / W;
    if (fabs(d) < mg) mg = fabs(d);
  }
  free(ord);
  if (margin) *margin = mg;
  return mg < ORC_AMBIG_EPS ? ORC_FLAG_TOPP_AMBIG : 0;
}

/* In place: keep prob >= min_p * max prob (src/sample/sampler.cpp:87-93).
 * *margin (if given) gets the smallest |w_i / min_p - 1| over the finite
 * entries, w_i = exp(z'_i - max z'). */
static int apply_min_p_m(float* zs, int V, float min_p, double* margin) {
  double mg = INFINITY;
  if (min_p > 0.0f) {
    float m = zs[0];
    for (int i = 1; i < V; ++i)
      if (zs[i] > m) m = zs[i];
    double W = 0.0;
    for (int i = 0; i < V; ++i) W += wexp(zs[i], m);
    const double thr = (1.0 / W) * (double)min_p; /* peak prob = 1/W */
    for (int i = 0; i < V; ++i) {
      if (zs[i] == -INFINITY) continue;
      const double w = wexp(zs[i], m);
      /* the max itself (w = 1) is kept for every min_p <= 1: no margin */
      if (zs[i] != m) {
        const double d = fabs(w / (double)min_p - 1.0);
        if (d < mg) mg = d;
      }
      if (w / W < thr) zs[i] = -INFINITY;
    }
  }
  if (margin) *margin = mg;
  return mg < ORC_AMBIG_EPS ? ORC_FLAG_MINP_AMBIG : 0;
}
void orc_apply_min_p(float* zs, int V, float min_p) { apply_min_p_m(zs, V, min_p, NULL); }

/* D4: inverse-CDF draw over the finite (kept) entries of zs, ascending index.
 * Replaces mx::random::categorical (src/sample/sampler.cpp:165). */
int orc_draw_row(const float* zs, int V, float u, double* margin) {
  float m = -INFINITY;
  for (int i = 0; i < V; ++i)
    if (zs[i] > m) m = zs[i];
  if (m == -INFINITY) {
    /* nothing left to draw (an all -inf row, or a top-p that rounds to 0):
     * MLX's categorical is the argmax of the logits plus Gumbel noise, -inf
     * everywhere, whose first index is 0 (D7) */
    if (margin) *margin = INFINITY;
    return 0;
  }
  double W = 0.0;
  for (int i = 0; i < V; ++i)
    if (zs[i] != -INFINITY) W += wexp(zs[i], m);
  if (!(u >= 0.0f)) u = 0.0f;
  if (u >= 1.0f) u = 0x1.fffffep-1f;
  const double target = (double)u * W;
  double cum = 0.0, prev = 0.0;
  int id = -1, last_pos = -1;
  for (int i = 0; i < V; ++i) {
    if (zs[i] == -INFINITY) continue;
    const double w = wexp(zs[i], m);
    if (w > 0.0) last_pos = i;
    prev = cum;
    cum += w;
    if (cum > target) {
      id = i;
      break;
    }
  }
  if (id < 0) { /* rounding left no crossing: last positive-weight entry */
    id = last_pos >= 0 ? last_pos : 0;
    prev = cum;
  }
  if (margin) {
    double a = (double)u - prev / W, b = cum / W - (double)u;
    *margin = a < b ? a : b;
  }
  return id;
}

/* ---- one row of Sampler::sample ------------------------------------------ */

typedef struct {
  int dtype;
  int K_max;
} orc_ctx;

static void sample_one_row(const void* row, const orc_ctx* c, int V, float T, int k, float p,
                           float mp, int tlp, float u, int32_t* id_out, float* lp_out, int32_t* top_ids,
                           float* top_lp, int32_t* flags_out, double* margins) {
  float* z = (float*)malloc(sizeof(float) * (size_t)V);
  for (int i = 0; i < V; ++i) z[i] = load_logit(row, c->dtype, (size_t)i);
  int flags = 0;
  double mg_p = INFINITY, mg_d = INFINITY;
  int id;

  /* Sanitisation as the C ABI does it (src/capi/mlxforge.cpp:55-60). */
  const int sampling = isfinite(T) && T > 0.0f && round_dtype(T, c->dtype) > 0.0f;
  if (!sampling) {
    id = orc_greedy_row(z, V); /* src/sample/sampler.cpp:156 */
    flags |= ORC_FLAG_GREEDY;
  } else {
    const float Tr = round_dtype(T, c->dtype); /* D1 */
    float* zs = (float*)malloc(sizeof(float) * (size_t)V);
    for (int i = 0; i < V; ++i) zs[i] = round_dtype(z[i] / Tr, c->dtype); /* :158 */
    if (k > 0) orc_apply_top_k(zs, V, k < V ? k : V);                      /* :159-161 */
    if (p > 0.0f && p < 1.0f) {                                            /* :162 */
      flags |= orc_apply_top_p(zs, V, round_dtype(p, c->dtype), &mg_p);    /* D6 */
    }
    if (mp > 0.0f && mp <= 1.0f)                                           /* :163, D9 */
      flags |= apply_min_p_m(zs, V, round_dtype(mp, c->dtype), NULL);
    id = orc_draw_row(zs, V, u, &mg_d); /* :165, D4 */
    if (mg_d < ORC_AMBIG_EPS) flags |= ORC_FLAG_DRAW_AMBIG;
    free(zs);
  }
  *id_out = id;

  /* Logprobs from the unscaled, unfiltered row (:146-154); rows with
   * top_logprobs < 0 are not computed (src/runtime/worker.cpp:477). */
  const int K_req = tlp > 0 ? (tlp < c->K_max ? tlp : c->K_max) : 0;
  const int K = K_req < V ? K_req : V;
  if (lp_out) {
    if (tlp >= 0) {
      const double lse = orc_lse_row(z, V);
      *lp_out = (float)((double)z[id] - lse);
      if (K > 0 && top_ids) {
        vi_t* ord = (vi_t*)malloc(sizeof(vi_t) * (size_t)V);
        for (int i = 0; i < V; ++i) {
          ord[i].v = z[i];
          ord[i].i = i;
        }
        qsort(ord, (size_t)V, sizeof(vi_t), cmp_desc_idx); /* argsort(-logp), :34 */
        for (int j = 0; j < K; ++j) {
          top_ids[j] = ord[j].i;
          top_lp[j] = (float)((double)ord[j].v - lse);
        }
        free(ord);
      }
    } else {
      *lp_out = NAN;
    }
  }
  if (top_ids)
    for (int j = K; j < c->K_max; ++j) {
      top_ids[j] = -1;
      top_lp[j] = -INFINITY;
    }
  if (flags_out) *flags_out = flags;
  if (margins) {
    margins[0] = mg_p;
    margins[1] = mg_d;
  }
  free(z);
}

/* ---- batched entry, threaded over rows ----------------------------------- */

typedef struct {
  const void* logits;
  const orc_ctx* c;
  int B, V;
  long row_stride;
  const float *T, *p, *mp, *u;
  const int *k, *tlp;
  int32_t* ids;
  float* lp;
  int32_t* top_ids;
  float* top_lp;
  int32_t* flags;
  double* margins;
  int next;
  pthread_mutex_t mu;
} orc_job;

static void* worker(void* arg) {
  orc_job* j = (orc_job*)arg;
  const size_t esz = j->c->dtype == ORC_F32 ? 4 : 2;
  for (;;) {
    pthread_mutex_lock(&j->mu);
    int r = j->next++;
    pthread_mutex_unlock(&j->mu);
    if (r >= j->B) break;
    const char* row = (const char*)j->logits + (size_t)r * (size_t)j->row_stride * esz;
    const int K_max = j->c->K_max;
    sample_one_row(row, j->c, j->V, j->T ? j->T[r] : 0.0f, j->k ? j->k[r] : 0,
                   j->p ? j->p[r] : 1.0f, j->mp ? j->mp[r] : 0.0f, j->tlp ? j->tlp[r] : -1,
                   j->u ? j->u[r] : 0.0f,
                   &j->ids[r], j->lp ? &j->lp[r] : NULL,
                   (j->top_ids && K_max > 0) ? &j->top_ids[(size_t)r * K_max] : NULL,
                   (j->top_lp && K_max > 0) ? &j->top_lp[(size_t)r * K_max] : NULL,
                   j->flags ? &j->flags[r] : NULL, j->margins ? &j->margins[2 * r] : NULL);
  }
  return NULL;
}

/* Batched oracle with the same argument meaning as the product's mlxf_sample_ex
 * (host pointers; min_p may be NULL).  Returns 0 on success, -1 on bad
 * arguments. */
int orc_sample_ex(const void* logits, int dtype, int B, int V, long row_stride, const float* T,
                  const int* k, const float* p, const float* min_p, const int* tlp, const float* u,
                  int32_t* ids, float* lp, int32_t* top_ids, float* top_lp, int K_max,
                  int32_t* flags, double* margins, int nthreads) {
  if (!logits || !ids || B < 0 || V <= 0 || row_stride < V || K_max < 0) return -1;
  if (dtype != ORC_F32 && dtype != ORC_BF16 && dtype != ORC_F16) return -1;
  orc_ctx c = {dtype, K_max};
  orc_job j;
  j.logits = logits;
  j.c = &c;
  j.B = B;
  j.V = V;
  j.row_stride = row_stride;
  j.T = T;
  j.k = k;
  j.p = p;
  j.mp = min_p;
  j.u = u;
  j.tlp = tlp;
  j.ids = ids;
  j.lp = lp;
  j.top_ids = top_ids;
  j.top_lp = top_lp;
  j.flags = flags;
  j.margins = margins;
  j.next = 0;
  pthread_mutex_init(&j.mu, NULL);
  if (nthreads < 1) nthreads = 1;
  if (nthreads > 256) nthreads = 256;
  pthread_t th[256];
  for (int t = 1; t < nthreads; ++t) pthread_create(&th[t], NULL, worker, &j);
  worker(&j);
  for (int t = 1; t < nthreads; ++t) pthread_join(th[t], NULL);
  pthread_mutex_destroy(&j.mu);
  return 0;
}

/* Penalties on one row in place (z holds values of the logits dtype):
 *   apply_repetition_penalty  src/sample/sampler.cpp:95-105
 *   apply_frequency_presence  src/sample/sampler.cpp:107-120
 *   penalize (order, when)    src/sample/sampler.cpp:122-133
 * with the C ABI's sanitisation (src/capi/mlxforge.cpp:59-64).  Every graph
 * op rounds to the logits dtype; the count of an id is its exact number of
 * occurrences, as a value of the dtype (D10).  Ids outside [0, V) are
 * ignored; NaN logits are left as they are. */
void orc_apply_penalties(float* z, int V, int dtype, const int* hist, int n, float rep, float freq,
                         float pres) {
  if (!(isfinite(rep) && rep > 0.0f)) rep = 1.0f;
  if (!isfinite(freq)) freq = 0.0f;
  if (!isfinite(pres)) pres = 0.0f;
  if (rep == 1.0f && freq == 0.0f && pres == 0.0f) return;
  unsigned* cnt = (unsigned*)calloc((size_t)V, sizeof(unsigned));
  for (int j = 0; j < n; ++j)
    if (hist[j] >= 0 && hist[j] < V) cnt[hist[j]]++;
  const float pen = round_dtype(rep, dtype), fq = round_dtype(freq, dtype), ps = round_dtype(pres, dtype);
  for (int i = 0; i < V; ++i) {
    if (!cnt[i] || isnan(z[i])) continue;
    float x = z[i];
    if (rep != 1.0f) x = x > 0.0f ? round_dtype(x / pen, dtype) : round_dtype(x * pen, dtype);
    if (freq != 0.0f || pres != 0.0f) {
      const float cd = round_dtype((float)cnt[i], dtype);
      x = round_dtype(x - round_dtype(cd * fq, dtype), dtype);
      x = round_dtype(x - ps, dtype);
    }
    z[i] = x;
  }
  free(cnt);
}

/* Philox4x32-10 (J. Salmon et al., "Parallel random numbers: as easy as 1,
 * 2, 3", SC'11): ten rounds of two 32x32->64 multiplies with the published
 * multipliers and Weyl key increments.  The draw uniform of a row is
 * (first word >> 8) * 2^-24 at key = seed, counter = (step, 0) -- the
 * product's replacement for the MLX key split per step
 * (src/runtime/worker.cpp:416,465-466). */
void orc_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
  uint32_t c0 = ctr[0], c1 = ctr[1], c2 = ctr[2], c3 = ctr[3], k0 = key[0], k1 = key[1];
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
    const uint32_t n0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0, n2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
    c0 = n0;
    c1 = (uint32_t)p1;
    c2 = n2;
    c3 = (uint32_t)p0;
    k0 += 0x9E3779B9u;
    k1 += 0xBB67AE85u;
  }
  out[0] = c0;
  out[1] = c1;
  out[2] = c2;
  out[3] = c3;
}

void orc_uniforms(int B, const uint64_t* seed, const uint64_t* step, float* u) {
  for (int r = 0; r < B; ++r) {
    const uint32_t ctr[4] = {(uint32_t)step[r], (uint32_t)(step[r] >> 32), 0u, 0u};
    const uint32_t key[2] = {(uint32_t)seed[r], (uint32_t)(seed[r] >> 32)};
    uint32_t o[4];
    orc_philox4x32_10(ctr, key, o);
    u[r] = (float)(o[0] >> 8) * 0x1p-24f;
  }
}

/* ---- admissible ids of an ambiguous row ---------------------------------- */

typedef struct {
  int32_t* out;
  int n, cap;
} idset;

static int idset_add(idset* s, int id) {
  for (int j = 0; j < s->n; ++j)
    if (s->out[j] == id) return 0;
  if (s->n >= s->cap) return -1;
  s->out[s->n++] = id;
  return 0;
}

/* Every id one row of Sampler::sample (src/sample/sampler.cpp:141-166, with
 * the decisions D1-D9) can return when the top-p threshold p, the draw
 * uniform u and the min_p threshold each move by up to eps (absolute for p and
 * u, relative for min_p): the checker for rows the ambiguity rule excludes
 * from the bit-exact comparison.
 *
 * After top-k (whose threshold is a comparison and never ambiguous), top-p and
 * min_p both keep a prefix of the (z' desc, index asc) order, so the kept set
 * is a prefix whose length L ranges over [L_lo, L_hi]; for each L the draw
 * (D4, ascending index) can return every kept element whose cumulative-mass
 * interval meets [(u - eps) W_L, (u + eps) W_L].  Writes the ids to out
 * (unordered) and returns their number; returns -1 when the range of L or of
 * the ids exceeds cap (the row cannot be checked), -2 on bad arguments. */
int orc_admissible(const void* row, int dtype, int V, float T, int k, float p, float mp, float u,
                   double eps, int32_t* out, int cap) {
  if (!row || !out || V <= 0 || cap <= 0) return -2;
  idset set = {out, 0, cap};
  float* z = (float*)malloc(sizeof(float) * (size_t)V);
  for (int i = 0; i < V; ++i) z[i] = load_logit(row, dtype, (size_t)i);
  const int sampling = isfinite(T) && T > 0.0f && round_dtype(T, dtype) > 0.0f;
  if (!sampling) {
    out[0] = orc_greedy_row(z, V);
    free(z);
    return 1;
  }
  const float Tr = round_dtype(T, dtype);
  float* zs = (float*)malloc(sizeof(float) * (size_t)V);
  for (int i = 0; i < V; ++i) zs[i] = round_dtype(z[i] / Tr, dtype);
  free(z);
  if (k > 0) orc_apply_top_k(zs, V, k < V ? k : V);
  vi_t* ord = (vi_t*)malloc(sizeof(vi_t) * (size_t)V);
  int N = 0;
  for (int i = 0; i < V; ++i)
    if (zs[i] != -INFINITY) {
      ord[N].v = zs[i];
      ord[N].i = i;
      ++N;
    }
  int rc = 0;
  if (N == 0) { /* nothing to draw: index 0 (D7) */
    idset_add(&set, 0);
    rc = 1;
    goto done;
  }
  qsort(ord, (size_t)N, sizeof(vi_t), cmp_desc_idx);
  {
    const float m = ord[0].v;
    double* w = (double*)malloc(sizeof(double) * (size_t)N);
    double* prior = (double*)malloc(sizeof(double) * (size_t)N);
    double W = 0.0;
    for (int j = 0; j < N; ++j) {
      w[j] = wexp(ord[j].v, m);
      prior[j] = W;
      W += w[j];
    }
    int n_lo = N, n_hi = N;
    if (p > 0.0f && p < 1.0f) {
      const double pc = (double)round_dtype(p, dtype);
      n_lo = n_hi = 0;
      for (int j = 0; j < N; ++j) {
        if (prior[j] < (pc - eps) * W) n_lo = j + 1;
        if (prior[j] < (pc + eps) * W) n_hi = j + 1;
      }
      if (pc > 0.0 && n_lo < 1) n_lo = 1;
      if (pc > 0.0 && n_hi < 1) n_hi = 1;
    }
    int m_lo = N, m_hi = N;
    if (mp > 0.0f && mp <= 1.0f) {
      const double mr = (double)round_dtype(mp, dtype);
      int ties = 0;
      m_lo = m_hi = 0;
      for (int j = 0; j < N; ++j) {
        if (w[j] >= mr * (1.0 + eps)) m_lo = j + 1;
        if (w[j] >= mr * (1.0 - eps)) m_hi = j + 1;
        if (ord[j].v == m) ties = j + 1;
      }
      if (m_lo < ties) m_lo = ties; /* the max's ties are always kept */
      if (m_hi < ties) m_hi = ties;
    }
    const int L_lo = n_lo < m_lo ? n_lo : m_lo;
    const int L_hi = n_hi < m_hi ? n_hi : m_hi;
    if (L_hi - L_lo > cap) {
      rc = -1;
    } else if (L_hi == 0) {
      idset_add(&set, 0); /* top-p rounded to 0: nothing kept */
      rc = 1;
    } else {
      int* rank = (int*)malloc(sizeof(int) * (size_t)V);
      for (int i = 0; i < V; ++i) rank[i] = -1;
      for (int j = 0; j < N; ++j) rank[ord[j].i] = j;
      float uc = u;
      if (!(uc >= 0.0f)) uc = 0.0f;
      if (uc >= 1.0f) uc = 0x1.fffffep-1f;
      for (int L = L_lo < 1 ? 1 : L_lo; L <= L_hi && rc >= 0; ++L) {
        double WL = 0.0;
        int last_pos = -1;
        for (int i = 0; i < V; ++i)
          if (rank[i] >= 0 && rank[i] < L) {
            WL += w[rank[i]];
            if (w[rank[i]] > 0.0) last_pos = i;
          }
        const double lo_t = ((double)uc - eps) * WL, hi_t = ((double)uc + eps) * WL;
        double C = 0.0;
        for (int i = 0; i < V && rc >= 0; ++i) {
          if (rank[i] < 0 || rank[i] >= L) continue;
          const double wi = w[rank[i]];
          if (wi <= 0.0) continue;
          const double prev = C;
          if (prev > hi_t) break;
          C += wi;
          if (C > lo_t && idset_add(&set, i)) rc = -1;
        }
        /* rounding can leave the target at or past the total: the last
         * positive-weight entry (orc_draw_row's fallback) */
        if (rc >= 0 && hi_t >= WL && last_pos >= 0 && idset_add(&set, last_pos)) rc = -1;
      }
      free(rank);
      if (rc >= 0) rc = set.n;
    }
    free(w);
    free(prior);
  }
done:
  free(ord);
  free(zs);
  return rc;
}

/* orc_sample_ex without min_p: the product's mlxf_sample. */
int orc_sample(const void* logits, int dtype, int B, int V, long row_stride, const float* T,
               const int* k, const float* p, const int* tlp, const float* u, int32_t* ids,
               float* lp, int32_t* top_ids, float* top_lp, int K_max, int32_t* flags,
               double* margins, int nthreads) {
  return orc_sample_ex(logits, dtype, B, V, row_stride, T, k, p, NULL, tlp, u, ids, lp, top_ids,
                       top_lp, K_max, flags, margins, nthreads);
}

/* Filter stage only (for the reference's filter known-answer tests and the
 * filter entry points): writes z' after temperature / top-k / top-p / min-p
 * into out (V floats).  Returns the ambiguity flags of the top-p and min_p
 * cutoffs (ORC_FLAG_TOPP_AMBIG, ORC_FLAG_MINP_AMBIG; see the exclusion rule
 * above), or -1 for bad arguments. */
int orc_filter_row(const float* zin, int V, int dtype, float T, int k, float p, float min_p,
                   float* out) {
  if (!zin || !out || V <= 0) return -1;
  const float Tr = round_dtype(T, dtype);
  /* the sampling call's sentinels: a temperature that is not a positive finite
   * value of the dtype divides nothing; min_p outside (0, 1] is off and inside
   * is rounded to the dtype (D9) */
  const int div = isfinite(T) && T > 0.0f && Tr > 0.0f;
  for (int i = 0; i < V; ++i) {
    float z = isnan(zin[i]) ? -INFINITY : zin[i];
    out[i] = div ? round_dtype(z / Tr, dtype) : z;
  }
  int flags = 0;
  if (k > 0) orc_apply_top_k(out, V, k);
  if (p > 0.0f && p < 1.0f) flags |= orc_apply_top_p(out, V, round_dtype(p, dtype), NULL);
  if (min_p > 0.0f && min_p <= 1.0f) flags |= apply_min_p_m(out, V, round_dtype(min_p, dtype), NULL);
  return flags;
}
