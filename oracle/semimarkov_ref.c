/*
 * semimarkov_ref.c -- plain-C restatement of the reference streaming semi-CRF
 * recursions (biobenkj/torch-semimarkov).  TEST INFRASTRUCTURE ONLY: it is
 * loaded by oracle/cref.py from tests/, the fixture generator under
 * tests/golden/ and bench.py's cpu_baseline leg, never by the product package.
 *
 * It exists because the PyTorch restatement (oracle/streaming_ref.py) is a
 * per-position Python loop that cannot reach the benchmark configurations
 * (T = 10^6 positions, or C = 128 with K = 500) in reasonable time.
 *
 * What it computes (paths relative to the reference's src/torch_semimarkov/):
 *   edge[s, k, c_dst, c_src] = (cum[s+k, c_dst] - cum[s, c_dst]) + db[min(k, K-1), c_dst]
 *                              (+ ps[s, c_dst]) (+ pe[s+k-1, c_dst]) + tr[c_src, c_dst]
 *                              (streaming/pytorch_reference.py:48-113)
 *   durations k = 1 .. max(min(K-1, t), 1); K = 1 means duration 1 with db row 0
 *   alpha[0, :] = 0, alpha[t, c] = (+)_{k, c'} alpha[t-k, c'] + edge[t-k, k, c, c']
 *                              (streaming/pytorch_reference.py:116-273)
 *   beta[len, :] = 0,  beta[t, c'] = (+)_{k, c} edge[t, k, c, c'] + beta[t+k, c]
 *   marginal m(t, k, c_dst, c_src) = exp(alpha[t, c_src] + edge + beta[t+k, c_dst] - logZ)
 *   grad_cum[t+k] += sum_src m, grad_cum[t] -= sum_src m, grad_tr += m^T,
 *   grad_db[min(k, K-1)] += sum_src m, grad_ps[t] += ..., grad_pe[t+k-1] += ...
 *                              (streaming/pytorch_reference.py:276-525)
 *   Viterbi: strict '>' over ascending k, first source label on ties, first
 *   final label on ties, backtrace to (start, end, label, prev)  (nn.py:444-531)
 *
 * How (fp64, smref_forward / smref_backward): the edge's source-label part is
 * the transition alone, so both sums factor exactly,
 *   u[s, c]     = (+)_{c'} alpha[s, c'] + tr[c', c]
 *   alpha[t, c] = (+)_k seg(t-k, k, c) + u[t-k, c]
 *   w[t, c]     = (+)_k seg(t, k, c) + beta[t+k, c]
 *   beta[t, c'] = (+)_c tr[c', c] + w[t, c]
 *   sum_src m(t, k, c, .) = exp(u[t, c] + seg(t, k, c) + beta[t+k, c] - logZ)
 *   grad_tr[c', c] = sum_t exp(alpha[t, c'] + tr[c', c] - u[t, c]) * sum_k (...)
 * which is the same function in exact arithmetic; in fp64 it agrees with the
 * direct K*C^2 recursion of oracle/streaming_ref.py to ~1e-12 relative
 * (tests/test_oracle.py pins it against that restatement on random problems,
 * projections, ragged and zero lengths and K = 1, and against its identities).
 *
 * The Viterbi routines run the DIRECT recursion (K*C^2 candidates per step):
 *   smref_viterbi_f32: the reference's fp32 operation order exactly
 *     (content = cum[t] - cum[s]; + db; + tr; alpha + edge, each rounded to
 *     fp32), so its table, score and segments are the reference's bit for bit;
 *   smref_viterbi_f64: the same in fp64, and for every (t, c) the gap between
 *     the best and the runner-up candidate (k, c'), so a caller can tell which
 *     inputs are tie-free: per sequence, the smallest gap over the decisions
 *     its backtrace takes (and the final-label decision).
 * Projections are not supported by the Viterbi routines (NULL only).
 *
 * Build: oracle/Makefile (gcc, OpenMP).  All arrays are host memory, dense
 * row-major; lengths are clamped to [0, T].
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#define SM_NEG_INF (-1e9) /* streaming/constants.py:10 */
#define SM_LOWEST (-1e300)

static inline int clampi(int64_t v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : (int)v); }

/* log-sum-exp (semiring 0) or max (semiring 1) of n values */
static double reduce_n(const double* a, int n, int semiring) {
  double m = SM_LOWEST;
  for (int i = 0; i < n; ++i) m = a[i] > m ? a[i] : m;
  if (semiring == 1 || n == 0) return m;
  double s = 0.0;
  for (int i = 0; i < n; ++i) s += exp(a[i] - m);
  return m + log(s);
}

/* segment score without the transition: content + db (+ ps) (+ pe) */
static inline double seg_score(const double* cum, const double* db, const double* ps, const double* pe, int C,
                               int K, int s, int k, int c) {
  const int kk = k < K - 1 ? k : K - 1;
  double v = (cum[(size_t)(s + k) * C + c] - cum[(size_t)s * C + c]) + db[(size_t)kk * C + c];
  if (ps) v += ps[(size_t)s * C + c];
  if (pe) v += pe[(size_t)(s + k - 1) * C + c];
  return v;
}

static inline int kmax_at(int K, int t) {
  if (K == 1) return 1;
  return t < K - 1 ? t : K - 1;
}

/* u[s, :] from alpha[s, :] */
static void mix_row(const double* arow, const double* tr, int C, int semiring, double* tmp, double* urow,
                    int c_lo, int c_hi) {
  for (int c = c_lo; c < c_hi; ++c) {
    for (int cp = 0; cp < C; ++cp) tmp[cp] = arow[cp] + tr[(size_t)cp * C + c];
    urow[c] = reduce_n(tmp, C, semiring);
  }
}

/* forward of one sequence: alpha (L+1, C) and u (L+1, C); returns the final reduction */
static double forward_one(const double* cum, const double* tr, const double* db, const double* ps,
                          const double* pe, int L, int C, int K, int semiring, double* alpha, double* u) {
  const int Kt = K == 1 ? 1 : K - 1;
  for (int c = 0; c < C; ++c) alpha[c] = 0.0;
#pragma omp parallel
  {
    double* tmp = (double*)malloc(sizeof(double) * (size_t)(C > Kt ? C : Kt));
    int nth = 1, id = 0;
#ifdef _OPENMP
    nth = omp_get_num_threads();
    id = omp_get_thread_num();
#endif
    const int c_lo = (int)((int64_t)C * id / nth), c_hi = (int)((int64_t)C * (id + 1) / nth);
    mix_row(alpha, tr, C, semiring, tmp, u, c_lo, c_hi);
#pragma omp barrier
    for (int t = 1; t <= L; ++t) {
      const int km = kmax_at(K, t);
      for (int c = c_lo; c < c_hi; ++c) {
        for (int k = 1; k <= km; ++k)
          tmp[k - 1] = u[(size_t)(t - k) * C + c] + seg_score(cum, db, ps, pe, C, K, t - k, k, c);
        alpha[(size_t)t * C + c] = reduce_n(tmp, km, semiring);
      }
#pragma omp barrier
      mix_row(alpha + (size_t)t * C, tr, C, semiring, tmp, u + (size_t)t * C, c_lo, c_hi);
#pragma omp barrier
    }
    free(tmp);
  }
  if (L == 0) {
    /* the reference's final row stays NEG_INF when no step reaches len = 0 */
    return semiring == 1 ? SM_NEG_INF : SM_NEG_INF + log((double)C);
  }
  return reduce_n(alpha + (size_t)L * C, C, semiring);
}

/*
 * Forward: logZ (B,) (log semiring) or the Viterbi score (max semiring).
 * alpha_out (B, T+1, C) may be NULL; rows past a sequence's length are NEG_INF.
 */
int smref_forward(const double* cum, const double* tr, const double* db, const int64_t* lengths, const double* ps,
                  const double* pe, int B, int T, int C, int K, int semiring, int nthreads, double* logZ,
                  double* alpha_out) {
  if (B < 1 || T < 1 || C < 1 || K < 1 || (semiring != 0 && semiring != 1)) return 1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
  const size_t rows = (size_t)(T + 1) * C;
  double* alpha = (double*)malloc(sizeof(double) * rows);
  double* u = (double*)malloc(sizeof(double) * rows);
  if (!alpha || !u) {
    free(alpha);
    free(u);
    return 2;
  }
  for (int b = 0; b < B; ++b) {
    const int L = clampi(lengths[b], 0, T);
    const double* cb = cum + (size_t)b * rows;
    const double* psb = ps ? ps + (size_t)b * T * C : NULL;
    const double* peb = pe ? pe + (size_t)b * T * C : NULL;
    logZ[b] = forward_one(cb, tr, db, psb, peb, L, C, K, semiring, alpha, u);
    if (alpha_out) {
      double* ao = alpha_out + (size_t)b * rows;
      memcpy(ao, alpha, sizeof(double) * (size_t)(L + 1) * C);
      for (size_t i = (size_t)(L + 1) * C; i < rows; ++i) ao[i] = SM_NEG_INF;
    }
  }
  free(alpha);
  free(u);
  return 0;
}

/*
 * Backward of the log partition (log semiring), per batch element (the
 * reference's per-sequence workspaces before the grad_output reduction):
 *   grad_cum (B, T+1, C), grad_tr (B, C, C), grad_db (B, K, C),
 *   grad_ps / grad_pe (B, T, C) or NULL (exactly when ps / pe are NULL),
 *   logZ (B,) the partition it used.
 * All outputs are fully written (zeros past each length).
 */
int smref_backward(const double* cum, const double* tr, const double* db, const int64_t* lengths, const double* ps,
                   const double* pe, int B, int T, int C, int K, int nthreads, double* logZ, double* grad_cum,
                   double* grad_tr, double* grad_db, double* grad_ps, double* grad_pe) {
  if (B < 1 || T < 1 || C < 1 || K < 1) return 1;
  if ((ps == NULL) != (grad_ps == NULL) || (pe == NULL) != (grad_pe == NULL)) return 1;
#ifdef _OPENMP
  if (nthreads > 0) omp_set_num_threads(nthreads);
#else
  (void)nthreads;
#endif
  const size_t rows = (size_t)(T + 1) * C;
  const int Kt = K == 1 ? 1 : K - 1;
  double* alpha = (double*)malloc(sizeof(double) * rows);
  double* u = (double*)malloc(sizeof(double) * rows);
  double* beta = (double*)malloc(sizeof(double) * rows);
  double* sst = (double*)malloc(sizeof(double) * rows);
  double* w = (double*)malloc(sizeof(double) * (size_t)C);
  if (!alpha || !u || !beta || !sst || !w) {
    free(alpha);
    free(u);
    free(beta);
    free(sst);
    free(w);
    return 2;
  }
  memset(grad_cum, 0, sizeof(double) * (size_t)B * rows);
  memset(grad_tr, 0, sizeof(double) * (size_t)B * C * C);
  memset(grad_db, 0, sizeof(double) * (size_t)B * K * C);
  if (grad_ps) memset(grad_ps, 0, sizeof(double) * (size_t)B * T * C);
  if (grad_pe) memset(grad_pe, 0, sizeof(double) * (size_t)B * T * C);
  for (int b = 0; b < B; ++b) {
    const int L = clampi(lengths[b], 0, T);
    const double* cb = cum + (size_t)b * rows;
    const double* psb = ps ? ps + (size_t)b * T * C : NULL;
    const double* peb = pe ? pe + (size_t)b * T * C : NULL;
    double* gc = grad_cum + (size_t)b * rows;
    double* gt = grad_tr + (size_t)b * C * C;
    double* gd = grad_db + (size_t)b * K * C;
    double* gps = grad_ps ? grad_ps + (size_t)b * T * C : NULL;
    double* gpe = grad_pe ? grad_pe + (size_t)b * T * C : NULL;
    const double Z = forward_one(cb, tr, db, psb, peb, L, C, K, 0, alpha, u);
    logZ[b] = Z;
    if (L == 0) continue;
    for (int c = 0; c < C; ++c) beta[(size_t)L * C + c] = 0.0;
#pragma omp parallel
    {
      double* tmp = (double*)malloc(sizeof(double) * (size_t)(C > Kt ? C : Kt));
      double* ex = (double*)malloc(sizeof(double) * (size_t)Kt);
      int nth = 1, id = 0;
#ifdef _OPENMP
      nth = omp_get_num_threads();
      id = omp_get_thread_num();
#endif
      const int c_lo = (int)((int64_t)C * id / nth), c_hi = (int)((int64_t)C * (id + 1) / nth);
      for (int t = L - 1; t >= 0; --t) {
        const int km = kmax_at(K, L - t);
        for (int c = c_lo; c < c_hi; ++c) {
          double m = SM_LOWEST;
          for (int k = 1; k <= km; ++k) {
            const double x = seg_score(cb, db, psb, peb, C, K, t, k, c) + beta[(size_t)(t + k) * C + c];
            tmp[k - 1] = x;
            m = x > m ? x : m;
          }
          double s = 0.0;
          for (int k = 0; k < km; ++k) {
            ex[k] = exp(tmp[k] - m);
            s += ex[k];
          }
          w[c] = m + log(s);
          /* marginals of the segments [t, t+k) with label c, summed over the source label */
          const double f = exp(m + u[(size_t)t * C + c] - Z);
          double st = 0.0;
          for (int k = 1; k <= km; ++k) {
            const double p = ex[k - 1] * f;
            const int kk = k < K - 1 ? k : K - 1;
            gc[(size_t)(t + k) * C + c] += p;
            gd[(size_t)kk * C + c] += p;
            if (gpe) gpe[(size_t)(t + k - 1) * C + c] += p;
            st += p;
          }
          gc[(size_t)t * C + c] -= st;
          if (gps) gps[(size_t)t * C + c] += st;
          sst[(size_t)t * C + c] = st;
        }
#pragma omp barrier
        for (int cp = c_lo; cp < c_hi; ++cp) {
          for (int c = 0; c < C; ++c) tmp[c] = tr[(size_t)cp * C + c] + w[c];
          beta[(size_t)t * C + cp] = reduce_n(tmp, C, 0);
        }
#pragma omp barrier
      }
      /* transition gradient: sum_t exp(alpha[t, c'] + tr[c', c] - u[t, c]) * S[t, c] */
      for (int cp = c_lo; cp < c_hi; ++cp)
        for (int c = 0; c < C; ++c) {
          const double trv = tr[(size_t)cp * C + c];
          double acc = 0.0;
          for (int t = 0; t < L; ++t)
            acc += exp(alpha[(size_t)t * C + cp] + trv - u[(size_t)t * C + c]) * sst[(size_t)t * C + c];
          gt[(size_t)cp * C + c] = acc;
        }
      free(tmp);
      free(ex);
    }
  }
  free(alpha);
  free(u);
  free(beta);
  free(sst);
  free(w);
  return 0;
}

/*
 * Viterbi with backtrace, direct recursion, one sequence per OpenMP thread.
 * Outputs per sequence b:
 *   score[b]             max_c alpha[len, c] (fp64 value of the REAL table)
 *   nseg[b]              number of segments
 *   segs[b, i, 0..3]     (start, end inclusive, label, previous label), first segment first
 *   min_gap[b]           smallest nonzero best-minus-runner-up gap over the backtrace's
 *                        decisions (fp64 routine only; 1e300 when there is no competitor);
 *                        the runner-up is the best candidate strictly below the best
 *   n_close[b]           number of those decisions with a nonzero gap < close_thr
 *   n_ties[b]            number of those decisions where another candidate equals the
 *                        best exactly (fp64 routine only).  With fp32-valued inputs the
 *                        fp64 sums of a few terms are exact, so these are the structural
 *                        ties: a run of one label cut into segments scores the same for
 *                        every order of its segment durations (the content telescopes,
 *                        the duration and transition terms commute).
 */
#define SM_DEFINE_VITERBI(NAME, REAL, TRACK_GAPS)                                                                 \
  int NAME(const REAL* cum, const REAL* tr, const REAL* db, const int64_t* lengths, int B, int T, int C, int K,    \
           int nthreads, double close_thr, double* score, int32_t* nseg, int32_t* segs, double* min_gap,          \
           int32_t* n_close, int32_t* n_ties) {                                                                    \
    if (B < 1 || T < 1 || C < 1 || K < 1) return 1;                                                               \
    int bad = 0;                                                                                                   \
    const size_t rows = (size_t)(T + 1) * C;                                                                       \
    _Pragma("omp parallel for schedule(dynamic, 1) num_threads(nthreads > 0 ? nthreads : 1) reduction(| : bad)") \
    for (int b = 0; b < B; ++b) {                                                                                  \
      const int L = clampi(lengths[b], 0, T);                                                                      \
      const REAL* cb = cum + (size_t)b * rows;                                                                     \
      REAL* alpha = (REAL*)malloc(sizeof(REAL) * (size_t)(L + 1) * C);                                             \
      int32_t* bpk = (int32_t*)calloc((size_t)(L + 1) * C, sizeof(int32_t));                                       \
      int32_t* bpc = (int32_t*)calloc((size_t)(L + 1) * C, sizeof(int32_t));                                       \
      double* gap = TRACK_GAPS ? (double*)malloc(sizeof(double) * (size_t)(L + 1) * C) : NULL;                    \
      unsigned char* tie = TRACK_GAPS ? (unsigned char*)calloc((size_t)(L + 1) * C, 1) : NULL;                    \
      if (!alpha || !bpk || !bpc || (TRACK_GAPS && (!gap || !tie))) {                                              \
        bad |= 1;                                                                                                  \
        free(alpha);                                                                                               \
        free(bpk);                                                                                                 \
        free(bpc);                                                                                                 \
        free(gap);                                                                                                 \
        free(tie);                                                                                                 \
        continue;                                                                                                  \
      }                                                                                                            \
      for (int c = 0; c < C; ++c) alpha[c] = (REAL)0;                                                              \
      for (int t = 1; t <= L; ++t) {                                                                               \
        const int km = kmax_at(K, t);                                                                              \
        for (int c = 0; c < C; ++c) {                                                                              \
          REAL best = (REAL)SM_NEG_INF;                                                                            \
          int bk = 0, bc = 0;                                                                                      \
          double v1 = SM_LOWEST, v2 = SM_LOWEST;                                                                   \
          int n1 = 0;                                                                                              \
          for (int k = 1; k <= km; ++k) {                                                                          \
            const int s = t - k;                                                                                   \
            const int kk = k < K - 1 ? k : K - 1;                                                                  \
            const REAL content = cb[(size_t)t * C + c] - cb[(size_t)s * C + c];                                    \
            const REAL segv = content + db[(size_t)kk * C + c];                                                    \
            REAL bs = 0;                                                                                           \
            int bcs = 0;                                                                                           \
            for (int cp = 0; cp < C; ++cp) {                                                                       \
              const REAL edge = segv + tr[(size_t)cp * C + c];                                                     \
              const REAL cand = alpha[(size_t)s * C + cp] + edge;                                                  \
              if (cp == 0 || cand > bs) {                                                                          \
                bs = cand;                                                                                         \
                bcs = cp;                                                                                          \
              }                                                                                                    \
              if (TRACK_GAPS) {                                                                                    \
                if ((double)cand > v1) {                                                                           \
                  v2 = v1;                                                                                         \
                  v1 = (double)cand;                                                                               \
                  n1 = 1;                                                                                          \
                } else if ((double)cand == v1) {                                                                   \
                  ++n1;                                                                                            \
                } else if ((double)cand > v2) {                                                                    \
                  v2 = (double)cand;                                                                               \
                }                                                                                                  \
              }                                                                                                    \
            }                                                                                                      \
            if (bs > best) {                                                                                       \
              best = bs;                                                                                           \
              bk = k;                                                                                              \
              bc = bcs;                                                                                            \
            }                                                                                                      \
          }                                                                                                        \
          alpha[(size_t)t * C + c] = best;                                                                         \
          bpk[(size_t)t * C + c] = bk;                                                                             \
          bpc[(size_t)t * C + c] = bc;                                                                             \
          if (TRACK_GAPS) {                                                                                        \
            gap[(size_t)t * C + c] = v2 <= SM_LOWEST ? 1e300 : v1 - v2;                                            \
            tie[(size_t)t * C + c] = n1 > 1 ? 1 : 0;                                                               \
          }                                                                                                        \
        }                                                                                                          \
      }                                                                                                            \
      /* final label: first maximum (argmax) */                                                                    \
      int cf = 0;                                                                                                  \
      double g_final = 1e300;                                                                                      \
      int t_final = 0;                                                                                             \
      if (L > 0) {                                                                                                 \
        double f1 = SM_LOWEST, f2 = SM_LOWEST;                                                                     \
        int nf = 0;                                                                                                \
        for (int c = 0; c < C; ++c) {                                                                              \
          const REAL v = alpha[(size_t)L * C + c];                                                                 \
          if (v > alpha[(size_t)L * C + cf]) cf = c;                                                               \
          if ((double)v > f1) {                                                                                    \
            f2 = f1;                                                                                               \
            f1 = (double)v;                                                                                        \
            nf = 1;                                                                                                \
          } else if ((double)v == f1) {                                                                            \
            ++nf;                                                                                                  \
          } else if ((double)v > f2) {                                                                             \
            f2 = (double)v;                                                                                        \
          }                                                                                                        \
        }                                                                                                          \
        if (f2 > SM_LOWEST) g_final = f1 - f2;                                                                     \
        t_final = nf > 1 ? 1 : 0;                                                                                  \
        score[b] = (double)alpha[(size_t)L * C + cf];                                                              \
      } else {                                                                                                     \
        score[b] = SM_NEG_INF;                                                                                     \
      }                                                                                                            \
      /* backtrace, last segment first, then reversed in place */                                                  \
      int32_t* sb = segs + (size_t)b * T * 4;                                                                      \
      int n = 0, t = L, c = cf;                                                                                    \
      double mg = g_final;                                                                                         \
      int n_cl = (TRACK_GAPS && L > 0 && g_final < close_thr) ? 1 : 0;                                            \
      int n_tie = TRACK_GAPS ? t_final : 0;                                                                        \
      while (t > 0) {                                                                                              \
        const int k = bpk[(size_t)t * C + c], cp = bpc[(size_t)t * C + c];                                         \
        if (k == 0) break;                                                                                         \
        if (TRACK_GAPS) {                                                                                          \
          const double g = gap[(size_t)t * C + c];                                                                 \
          mg = g < mg ? g : mg;                                                                                    \
          n_cl += g < close_thr ? 1 : 0;                                                                          \
          n_tie += tie[(size_t)t * C + c];                                                                         \
        }                                                                                                          \
        sb[4 * n + 0] = t - k;                                                                                     \
        sb[4 * n + 1] = t - 1;                                                                                     \
        sb[4 * n + 2] = c;                                                                                         \
        sb[4 * n + 3] = cp;                                                                                        \
        ++n;                                                                                                       \
        t -= k;                                                                                                    \
        c = cp;                                                                                                    \
      }                                                                                                            \
      for (int i = 0; i < n / 2; ++i)                                                                              \
        for (int j = 0; j < 4; ++j) {                                                                              \
          const int32_t x = sb[4 * i + j];                                                                         \
          sb[4 * i + j] = sb[4 * (n - 1 - i) + j];                                                                 \
          sb[4 * (n - 1 - i) + j] = x;                                                                             \
        }                                                                                                          \
      nseg[b] = n;                                                                                                 \
      if (min_gap) min_gap[b] = TRACK_GAPS ? mg : 0.0;                                                            \
      if (n_close) n_close[b] = n_cl;                                                                             \
      if (n_ties) n_ties[b] = n_tie;                                                                               \
      free(alpha);                                                                                                 \
      free(bpk);                                                                                                   \
      free(bpc);                                                                                                   \
      free(gap);                                                                                                   \
      free(tie);                                                                                                   \
    }                                                                                                              \
    return bad ? 2 : 0;                                                                                            \
  }

SM_DEFINE_VITERBI(smref_viterbi_f32, float, 0)
SM_DEFINE_VITERBI(smref_viterbi_f64, double, 1)

int smref_version(void) { return 1; }
