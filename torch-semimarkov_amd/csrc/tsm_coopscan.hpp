// Cooperative register-resident log-semiring scan for label sets whose rings do
// not fit one CU's LDS (C up to 128 with long durations: C * Kmax fp64 ring
// entries = 512 KB at C = 128, K = 500).
//
// A chunk of a sequence is scanned by a group of G workgroups; member m owns
// the CL = ceil(C / G) labels [m*CL, (m+1)*CL) and keeps only their rings in
// LDS.  Each step runs the register-resident pull of tsm_fastscan.hpp for the
// member's own labels (16 lanes per label, R durations per lane), then the
// group exchanges its row of results through global memory: every result is
// one 64-bit word (fp32 value | 32-bit step stamp) stored with a relaxed
// agent-scope atomic, and every member polls the C words of the step until
// all carry the step's stamp.  The value travels with its stamp, so no fence
// is needed.  The stamp is a per-group step counter that grows over the whole
// launch (the buffer is cleared before each launch), so a stale word never
// matches.  With the full row in LDS every member computes the normaliser and
// the label mix of its own labels exactly as the single-workgroup scan does.
//
// Launches are cooperative (all groups co-resident) and persistent: NQ groups
// loop over the chunks.  Members of a group take block ids with equal
// blockIdx % 8 when the CU count allows it, which the dispatcher places on one
// XCD (one L2).  Every poll is bounded: past the limit (or once another block
// gave up) a block sets the abort flag and leaves, and the repair kernel then
// poisons the result with NaN instead of hanging.
//
// Chunking, speculation, verification (verify_kernel), retry, sequential
// repair and level offsets follow tsm_chunk_driver.hpp, with groups in place
// of blocks.
#pragma once

#include <float.h>

#include <algorithm>

#include "tsm_chunk_driver.hpp"

namespace tsm {
namespace coop {

using namespace scan_detail;

constexpr double kInvD = -1e30;
constexpr double kLog2eD = 1.4426950408889634;
constexpr int kSpinLimit = 1 << 22;  // polls of one word before giving up (seconds)

__device__ __forceinline__ void lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
__device__ __forceinline__ void wave_lds_order() { __asm__ volatile("" ::: "memory"); }

// Group and member of a block.  xmap: members share blockIdx % 8.
struct Member {
  int q, m;
  bool valid;
};

__device__ __forceinline__ Member member_of(const ScanParams& p) {
  const int bid = blockIdx.x;
  Member r;
  if (p.xmap) {
    const int x = bid & 7, w = bid >> 3;
    r.m = w % p.G;
    r.q = (w / p.G) * 8 + x;
  } else {
    r.m = bid % p.G;
    r.q = bid / p.G;
  }
  r.valid = r.q < p.NQ;
  return r;
}

__device__ __forceinline__ bool aborted(const ScanParams& p) {
  return __hip_atomic_load(p.xabort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != 0;
}

// Writes this member's result of step s into the group's slot of the step's parity.
__device__ __forceinline__ void publish_row(const ScanParams& p, unsigned long long* xb, unsigned s, bool writer,
                                            int c, float a2) {
  if (writer) {
    const unsigned long long w = ((unsigned long long)s << 32) | (unsigned long long)__float_as_uint(a2);
    __hip_atomic_store(&xb[(s & 1) * p.C + c], w, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Gathers the group's full row of step s into row[0..C).  All threads call it;
// false when the group gave up.
__device__ inline bool gather_row(const ScanParams& p, unsigned long long* xb, unsigned s, float* row, int* sflag) {
  const int C = p.C, par = s & 1;
  for (int cc = threadIdx.x; cc < C; cc += blockDim.x) {
    unsigned long long w;
    int n = 0;
    for (;;) {
      w = __hip_atomic_load(&xb[par * C + cc], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((unsigned)(w >> 32) == s) break;
      ++n;
      if (n > kSpinLimit || ((n & 1023) == 0 && aborted(p))) {
        __hip_atomic_store(p.xabort, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *sflag = 1;
        break;
      }
    }
    row[cc] = __uint_as_float((unsigned)w);
  }
  lds_barrier();
  return *sflag == 0;
}

// Writes this member's results of step s and gathers the group's full row of
// step s into row[0..C).  All threads call it; false when the group gave up.
__device__ inline bool exchange_row(const ScanParams& p, unsigned long long* xb, unsigned s, bool writer, int c,
                                    float a2, float* row, int* sflag) {
  publish_row(p, xb, s, writer, c, a2);
  return gather_row(p, xb, s, row, sflag);
}

// LOGSR: log-sum-exp over durations and source labels; else max-plus, with the
// factorised Viterbi's backpointers `(k << 16) | c'` per (t, c) when p.bp is set
// (ties to the smallest duration, then the smallest source label, as the
// single-workgroup scan).
template <int J, int R, int CJ, bool FWD, bool LOGSR = true>
struct CoopChunk {
  static constexpr bool kFwd = FWD;
  static constexpr bool kLog = LOGSR;
  // register budget: a lane holds 2R fp64 terms (ring reads, duration biases)
  static constexpr int kMaxThreads = R > 16 ? 256 : 512;
  __device__ static double* red(char* smem, const ScanParams& p) {
    return reinterpret_cast<double*>(smem + coop_lds_layout(p.CL, p.C, p.RL, p.RS).red);
  }
  // One chunk of one sequence, this member's labels (modes as Chunk::run in
  // tsm_fastscan.hpp).  s: the group's step counter.  False when the group gave up.
  __device__ static bool run(const ScanParams& p, char* smem, int b, int j, int mode, const float* init_st,
                             const double* init_lv, int m, unsigned long long* xb, unsigned& s) {
    constexpr int KP = J * R;
    const int C = p.C, Kmax = p.Kmax, K = p.K, RS = p.RS, RL = p.RL, T = p.T, CL = p.CL;
    const int len = seq_len(p, b);
    const int item = b * p.P + j;
    const CoopLds L = coop_lds_layout(CL, C, RL, RS);
    double* ring = reinterpret_cast<double*>(smem + L.ring);
    double* lring = reinterpret_cast<double*>(smem + L.lring);
    float* row = reinterpret_cast<float*>(smem + L.row);
    int* sflag = reinterpret_cast<int*>(smem + L.flag);
    const int tid = threadIdx.x, NT = blockDim.x;
    const int c_lo = m * CL;
    const int CLv = min(CL, C - c_lo);  // labels this member owns
    const int g = tid / J, lj = tid % J;
    const bool cval = g < CLv;
    const int gl = cval ? g : CLv - 1;  // padding groups shadow the last own label and never write
    const int c = c_lo + gl;
    const bool lead = m == 0;  // writes the outputs every member computes identically
    const float* cum_b = p.cum + (size_t)b * (T + 1) * C;
    const bool has_ps = p.ps != nullptr, has_pe = p.pe != nullptr;
    const float* ps_b = has_ps ? p.ps + (size_t)b * T * C : nullptr;
    const float* pe_b = has_pe ? p.pe + (size_t)b * T * C : nullptr;
    const bool store = p.val != nullptr;
    const double sgn = FWD ? 1.0 : -1.0;
    auto cumx = [&](int pos) { return sgn * (double)cum_b[(size_t)pos * C + c] * kLog2eD; };

    int t_lo, t_hi, t_start, jl = 0;
    if (FWD) {
      t_lo = j * p.Lc;
      t_hi = min(t_lo + p.Lc, len);
      t_start = mode == 0 ? 0 : (mode == 1 ? t_lo - p.W : t_lo);
    } else {
      jl = bwd_last_chunk(p, len);
      t_lo = j * p.Lc;
      t_hi = (j == jl) ? len : (j + 1) * p.Lc;
      t_start = mode == 0 ? len : (mode == 1 ? t_hi + p.W : t_hi);
    }

    // ---- per-lane constants ----
    double dbr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int k = 1 + lj + J * r;
      const int di = k < K - 1 ? k : K - 1;
      dbr[r] = (k <= Kmax) ? (double)(p.db[(size_t)di * C + c] * kLog2e) : kInvD;
    }
    float trr[CJ];
#pragma unroll
    for (int i = 0; i < CJ; ++i) {
      const int ci = lj + J * i;
      trr[i] = (ci < C) ? (FWD ? p.trans[(size_t)ci * C + c] : p.trans[(size_t)c * C + ci]) * kLog2e : 0.0f;
    }
    // duration-bias factors relative to the lane's first duration (as in Chunk::run)
    float edb[R];
    bool lane_exact = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const double d = dbr[r] - dbr[0];
      edb[r] = exp2_hw((float)d);
      lane_exact = lane_exact || (d > 64.0);
    }

    // ---- empty rings ----
    for (int idx = tid; idx < CL * RL; idx += NT) ring[idx] = kInvD;
    for (int i = tid; i < RS; i += NT) lring[i] = 0.0;
    if (tid == 0) *sflag = 0;
    __syncthreads();

    double* rc = ring + (size_t)gl * RL;
    // linear ring as in Chunk::run: position t_start at A0, compaction to the top
    const int A0 = RL - KP;
    double lvl_prev;
    // ---- initial state ----
    if (mode == 0) {
      const int pos = t_start;  // FWD: 0, BWD: len
      lvl_prev = 0.0;
      float v0;
      if (FWD) {
        float mm = kMinusInf;
        [[maybe_unused]] int mi = 0x7fffffff;
        if constexpr (LOGSR) {
#pragma unroll
          for (int i = 0; i < CJ; ++i)
            if (lj + J * i < C) mm = fmax2(mm, trr[i]);
        } else {
#pragma unroll
          for (int i = 0; i < CJ; ++i)
            if (lj + J * i < C && trr[i] > mm) {
              mm = trr[i];
              mi = lj + J * i;
            }
        }
        float u0;
        if constexpr (LOGSR) {
          float sm = 0.0f;
#pragma unroll
          for (int i = 0; i < CJ; ++i)
            if (lj + J * i < C) sm += exp2_hw(trr[i] - mm);
          u0 = group_lse2<J>(mm, sm);
        } else {
          // best source label of a segment starting at position 0
          const ValIdx best = group_argmax_first<J>(ValIdx{mm, mi});
          u0 = best.v;
          if (p.bp != nullptr && cval && lj == 0 && j == 0) p.bp[((size_t)b * (T + 1)) * C + c] = best.i;
        }
        v0 = u0 + ((has_ps && T > 0) ? ps_b[c] * kLog2e : 0.0f);
        if (lead && g == 0) {
#pragma unroll
          for (int i = 0; i < CJ; ++i) {
            const int ci = lj + J * i;
            if (ci < C) {
              if (store && j == 0) p.val[((size_t)b * (T + 1)) * C + ci] = 0.0f;
              if (len == 0) p.fin[(size_t)b * C + ci] = 0.0f;
            }
          }
        }
        if (lead && tid == 0) {
          if (store && j == 0) p.lvl[(size_t)b * (T + 1)] = 0.0;
          if (len == 0) p.fin_lvl[b] = 0.0;
        }
      } else {
        v0 = (has_pe && len >= 1) ? pe_b[(size_t)(len - 1) * C + c] * kLog2e : 0.0f;
        if (cval && lj == 0 && store) p.val[((size_t)b * (T + 1) + len) * C + c] = 0.0f;
        if (lead && tid == 0 && store) p.lvl[(size_t)b * (T + 1) + len] = 0.0;
      }
      if (cval && lj == 0) rc[A0] = (double)v0 - cumx(pos);
      if (tid == 0) lring[pos % RS] = 0.0;
    } else {
      lvl_prev = (mode == 1) ? 0.0 : init_lv[0];
      if (cval) {
        for (int i = lj; i < Kmax; i += J) {
          const int pos = FWD ? t_start - i : t_start + i;
          float v;
          if (mode == 1) {
            if (FWD) v = has_ps ? ps_b[(size_t)pos * C + c] * kLog2e : 0.0f;
            else v = has_pe ? pe_b[(size_t)(pos - 1) * C + c] * kLog2e : 0.0f;
          } else {
            v = init_st[(size_t)i * C + c];
          }
          const double lv = (mode == 1) ? 0.0 : init_lv[i];
          rc[A0 + i] = lv + (double)v - cumx(pos);
        }
      }
      for (int i = tid; i < Kmax; i += NT) {
        const int pos = FWD ? t_start - i : t_start + i;
        lring[pos % RS] = (mode == 1) ? 0.0 : init_lv[i];
      }
    }
    __syncthreads();

    // ---- per-step operands, prefetched one step ahead ----
    const int dir = FWD ? 1 : -1;
    const int t_first = t_start + dir;
    const int t_end = FWD ? t_hi + 1 : t_lo - 1;  // exclusive
    auto clampT = [&](int t) { return t < 0 ? 0 : (t > T ? T : t); };
    auto clampT1 = [&](int t) { return t < 0 ? 0 : (t > T - 1 ? T - 1 : t); };
    const float* pa_src = FWD ? (has_pe ? pe_b : cum_b) : (has_ps ? ps_b : cum_b);
    const float* pb_src = FWD ? (has_ps ? ps_b : cum_b) : (has_pe ? pe_b : cum_b);
    const float pa_scale = (FWD ? has_pe : has_ps) ? kLog2e : 0.0f;
    const float pb_scale = (FWD ? has_ps : has_pe) ? kLog2e : 0.0f;
    auto pa_row = [&](int t) { return FWD ? clampT1(t - 1) : clampT1(t); };
    auto pb_row = [&](int t) { return FWD ? clampT1(t) : clampT1(t - 1); };
    // absent projections are not read (operand 0, scale 0)
    const bool has_pa = FWD ? has_pe : has_ps, has_pb = FWD ? has_ps : has_pe;
    float cum_n = cum_b[(size_t)clampT(t_first) * C + c];
    float pa_n = has_pa ? pa_src[(size_t)pa_row(t_first) * C + c] : 0.0f;
    float pb_n = has_pb ? pb_src[(size_t)pb_row(t_first) * C + c] : 0.0f;

    const int rec_spec = (mode == 1) ? (FWD ? t_lo : t_hi) : -1;
    const int rec_end = FWD ? ((t_hi < len) ? t_hi : -1) : ((j >= 1) ? t_lo : -1);

    // The pull of step t+1 over durations of register r >= 1 reads positions that
    // exist before step t's row comes back, so it runs while the row travels
    // between the members (the exchange is most of a step): psum = sum over
    // r >= 1 of 2^(e[r] - e[1]) * edb[r] (log), or the best of those terms (max).
    // The next step adds the register-0 terms (durations 1..16; the first is the
    // position step t writes).  `base` points at the next step's r = 0 entries.
    [[maybe_unused]] float psum = 0.0f;
    [[maybe_unused]] double pe1 = 0.0, pmax = 0.0;
    [[maybe_unused]] int pk = 0;
    auto partial_pull = [&](const double* base) {
      if constexpr (LOGSR) {
        pe1 = base[J];
        float q0 = edb[1], q1 = 0.0f;
#pragma unroll
        for (int r = 2; r < R; ++r) {
          const float x = exp2_hw((float)(base[J * r] - pe1));
          if (r & 1) q1 = fmaf(x, edb[r], q1);
          else q0 = fmaf(x, edb[r], q0);
        }
        psum = q0 + q1;
      } else {
        pmax = base[J] + dbr[1];
        pk = 1 + lj + J;
#pragma unroll
        for (int r = 2; r < R; ++r) {
          const double y = base[J * r] + dbr[r];
          if (y > pmax) {
            pmax = y;
            pk = 1 + lj + J * r;
          }
        }
      }
    };

    int A = A0;  // ring index of the current position
    partial_pull(rc + A0 + lj);  // step t_first: index A0 - 1, entries from A0 on
    for (int t = t_first; t != t_end; t += dir) {
      if (--A < 0) {
        if (cval) {
          double cp[R];
#pragma unroll
          for (int r = 0; r < R; ++r) cp[r] = rc[lj + J * r];
          wave_lds_order();
#pragma unroll
          for (int r = 0; r < R; ++r) rc[A0 + lj + J * r] = cp[r];
          wave_lds_order();
        }
        A = A0 - 1;
      }
      const double cx_t = sgn * (double)cum_n * kLog2eD;
      const float pa_t = pa_n * ((FWD ? t >= 1 : true) ? pa_scale : 0.0f);
      const float pb_t = pb_n * ((FWD ? true : t >= 1) ? pb_scale : 0.0f);
      {
        const int tn = t + dir;
        cum_n = cum_b[(size_t)clampT(tn) * C + c];
        if (has_pa) pa_n = pa_src[(size_t)pa_row(tn) * C + c];
        if (has_pb) pb_n = pb_src[(size_t)pb_row(tn) * C + c];
      }

      // ---- pull over the lane's durations (own labels): the register-0 terms
      //      and the partial sums of the others, computed during the last exchange ----
      const double* rb = rc + A + 1 + lj;
      const double e0 = rb[0];
      float a2;
      [[maybe_unused]] int kbest = 0;
      if constexpr (LOGSR) {
        double y0 = e0 + dbr[0];
        // 1 + 2^(e[1] - e[0]) * psum: the one-pass sum relative to the first term
        float sacc = fmaf(exp2_hw((float)(pe1 - e0)), psum, 1.0f);
        // overflow, extreme factors, or a partial sum so large that an underflowed
        // 2^(e[1] - e[0]) could still matter: the exact two-pass form
        if (__ballot(!(sacc <= FLT_MAX) || lane_exact || !(psum <= 0x1p64f))) {
          double e[R];
#pragma unroll
          for (int r = 0; r < R; ++r) e[r] = rb[J * r];
          double mx2 = y0;
#pragma unroll
          for (int r = 1; r < R; ++r) mx2 = fmax(mx2, e[r] + dbr[r]);
          sacc = 0.0f;
#pragma unroll
          for (int r = 0; r < R; ++r) sacc += exp2_hw((float)((e[r] + dbr[r]) - mx2));
          y0 = mx2;
        }
        a2 = group_lse2<J>((float)((y0 + cx_t) - lvl_prev), sacc) + pa_t;
      } else {
        // max over durations; ties go to the smallest duration (lanes hold ascending
        // k; register 0 holds the lane's smallest)
        double ym = e0 + dbr[0];
        int km = 1 + lj;
        if (pmax > ym) {
          ym = pmax;
          km = pk;
        }
        const ValIdx best = group_argmax_first<J>(ValIdx{(float)((ym + cx_t) - lvl_prev), km});
        a2 = best.v + pa_t;
        kbest = best.i;
      }

      // ---- the group's row of all labels; the next step's partial pull meanwhile
      //      (its index A - 1: entries from A on; every one exists already) ----
      ++s;
      const int par = s & 1;
      publish_row(p, xb, s, cval && lj == 0, c, a2);
      partial_pull(rc + A + lj);
      if (!gather_row(p, xb, s, row + par * C, sflag)) return false;

      // ---- all labels: normaliser and label mix of the own labels ----
      float rv[CJ];
      float ml = kMinusInf;
#pragma unroll
      for (int i = 0; i < CJ; ++i) {
        const int ci = lj + J * i;
        rv[i] = (ci < C) ? row[par * C + ci] : kMinusInf;
        ml = fmax2(ml, rv[i]);
      }
      const float mx = group_max<J>(ml);
      const double lvl_t = lvl_prev + (double)mx;
      float mixv;
      if constexpr (LOGSR) {
        float mq = kMinusInf;
#pragma unroll
        for (int i = 0; i < CJ; ++i)
          if (lj + J * i < C) mq = fmax2(mq, (rv[i] - mx) + trr[i]);
        float sq = 0.0f;
#pragma unroll
        for (int i = 0; i < CJ; ++i)
          if (lj + J * i < C) sq += exp2_hw(((rv[i] - mx) + trr[i]) - mq);
        mixv = group_lse2<J>(mq, sq);
      } else {
        float mq = kMinusInf;
        int mqi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < CJ; ++i)
          if (lj + J * i < C) {
            const float q = (rv[i] - mx) + trr[i];
            if (q > mq) {
              mq = q;
              mqi = lj + J * i;
            }
          }
        // best source label for a segment starting at t (first on ties)
        const ValIdx best = group_argmax_first<J>(ValIdx{mq, mqi});
        mixv = best.v;
        if (FWD && p.bp != nullptr && cval && lj == 0 && (j == 0 || t > t_lo))
          p.bp[((size_t)b * (T + 1) + t) * C + c] = (kbest << 16) | best.i;
      }

      const bool owned = FWD ? (j == 0 || t > t_lo) : (t < t_hi || j == jl);
      if (FWD) {
        if (lead && g == 0) {
#pragma unroll
          for (int i = 0; i < CJ; ++i) {
            const int ci = lj + J * i;
            if (ci < C) {
              const float ah = rv[i] - mx;
              if (store && owned) p.val[((size_t)b * (T + 1) + t) * C + ci] = ah;
              if (t == len) p.fin[(size_t)b * C + ci] = ah;
            }
          }
        }
        if (lead && tid == 0) {
          if (store && owned) p.lvl[(size_t)b * (T + 1) + t] = lvl_t;
          if (t == len) p.fin_lvl[b] = lvl_t;
        }
      } else {
        if (cval && lj == 0 && store && owned) p.val[((size_t)b * (T + 1) + t) * C + c] = mixv;
        if (lead && tid == 0 && store && owned) p.lvl[(size_t)b * (T + 1) + t] = lvl_t;
      }
      // ---- ring entry for position t ----
      if (cval && lj == 0) rc[A] = (lvl_t + (double)(mixv + pb_t)) - cx_t;
      if (tid == 0) lring[t % RS] = lvl_t;
      lvl_prev = lvl_t;
      wave_lds_order();

      // ---- boundary states for verification: positions t -/+ i, i < Kmax ----
      if (t == rec_spec || t == rec_end) {
        float* st = (t == rec_spec ? p.st_spec : p.st_end) + (size_t)item * Kmax * C;
        double* lv = (t == rec_spec ? p.lv_spec : p.lv_end) + (size_t)item * Kmax;
        if (cval) {
          for (int i = lj; i < Kmax; i += J) {
            const int pos = FWD ? t - i : t + i;
            const double x = rc[A + i];
            const double lp = (i == 0) ? lvl_t : lring[pos % RS];
            st[(size_t)i * C + c] = (x < -1e29) ? -1e30f : (float)((x - lp) + cumx(pos));
          }
        }
        if (lead) {
          for (int i = tid; i < Kmax; i += NT) {
            const int pos = FWD ? t - i : t + i;
            lv[i] = (i == 0) ? lvl_t : lring[pos % RS];
          }
        }
      }
    }
    return true;
  }
};

// Parallel pass (main or retry) over all chunks, one group per chunk at a time.
template <class CH>
__device__ __forceinline__ void coop_scan_body(const ScanParams& p) {
  extern __shared__ __align__(16) char smem[];
  constexpr bool FWD = CH::kFwd;
  const Member me = member_of(p);
  if (!me.valid) return;
  unsigned long long* xb = p.xch + (size_t)me.q * 2 * p.C;
  unsigned s = 0;
  const bool lead = me.m == 0;
  for (int item = me.q; item < p.B * p.P; item += p.NQ) {
    const int b = item / p.P, j = item % p.P;
    const int len = seq_len(p, b);
    if (FWD ? (j > 0 && j * p.Lc >= len) : (j > bwd_last_chunk(p, len))) {
      if (lead && threadIdx.x == 0) p.status[item] = -1;  // empty chunk
      continue;
    }
    // every member reads the status before any member rewrites it: the rewrite
    // follows the chunk's steps, and no member passes a step's exchange alone
    if (p.retry && !(p.status[item] == 1 && (p.vstat[2 * item] - p.vstat[2 * item + 1] > (double)p.tol))) continue;
    const int mode = (FWD ? fwd_spec(p, j) : bwd_spec(p, j, len)) ? 1 : 0;
    if (!CH::run(p, smem, b, j, mode, nullptr, nullptr, me.m, xb, s)) return;
    if (lead && threadIdx.x == 0) {
      p.status[item] = mode;
      if (p.retry) *p.vflag = 1;
    }
    __syncthreads();
  }
}

template <class CH>
__global__ void __launch_bounds__(CH::kMaxThreads) coop_scan_kernel(ScanParams p) {
  coop_scan_body<CH>(p);
}

template <class CH>
__global__ void __launch_bounds__(CH::kMaxThreads) coop_retry_kernel(ScanParams p) {
  coop_scan_body<CH>(p);
}

// Sequential verification / repair (chunk_fixup_kernel with groups): one group
// per sequence at a time.  A recomputed chunk's boundary state is written by
// every member (its own labels) and read whole by the next step of the walk,
// so members fence before moving on.  An earlier give-up poisons the result.
template <class CH>
__global__ void __launch_bounds__(CH::kMaxThreads) coop_fixup_kernel(ScanParams p) {
  extern __shared__ __align__(16) char smem[];
  constexpr bool FWD = CH::kFwd;
  const Member me = member_of(p);
  if (!me.valid) return;
  unsigned long long* xb = p.xch + (size_t)me.q * 2 * p.C;
  unsigned s = 0;
  const bool lead = me.m == 0;
  double* red = CH::red(smem, p);
  const int Kmax = p.Kmax, C = p.C;
  const CoopLds L = coop_lds_layout(p.CL, C, p.RL, p.RS);
  float* row = reinterpret_cast<float*>(smem + L.row);
  int* sflag = reinterpret_cast<int*>(smem + L.flag);
  const int c_lo = me.m * p.CL, CLv = min(p.CL, C - c_lo);
  for (int b = me.q; b < p.B; b += p.NQ) {
    const int len = seq_len(p, b);
    double F = aborted(p) ? __builtin_nan("") : 0.0;
    int n_re = 0;
    bool prev_recomputed = false;
    const int jl = bwd_last_chunk(p, len);
    const int nch = len == 0 ? 1 : (len + p.Lc - 1) / p.Lc;
    if (lead && threadIdx.x == 0) p.offs[(size_t)b * p.P + (FWD ? 0 : jl)] = 0.0;
    for (int j = FWD ? 1 : jl - 1; FWD ? j < nch : j >= 0; j += FWD ? 1 : -1) {
      const int item = b * p.P + j;
      if (p.status[item] != 1) {
        F = aborted(p) ? __builtin_nan("") : 0.0;  // the chunk ran exactly from the sequence end
        prev_recomputed = false;
      } else {
        const size_t e = FWD ? (size_t)(item - 1) : (size_t)(item + 1), sp = (size_t)item;
        double dmax, dmin;
        if (!prev_recomputed) {
          dmax = p.vstat[2 * sp];
          dmin = p.vstat[2 * sp + 1];
        } else {
          double hi, lo;
          boundary_spread_part(p, e, sp, hi, lo);
          block_minmax(hi, lo, red, dmax, dmin);
        }
        if (dmax - dmin <= (double)p.tol) {
          F += 0.5 * (dmax + dmin);
          prev_recomputed = false;
        } else {
          if (!CH::run(p, smem, b, j, 2, p.st_end + e * Kmax * C, p.lv_end + e * Kmax, me.m, xb, s)) {
            F = __builtin_nan("");
          }
          __threadfence();  // this member's boundary columns before the others read them
          __syncthreads();
          ++n_re;
          prev_recomputed = true;
          if (lead && threadIdx.x == 0) p.status[item] = 2;
          // all members' boundary columns are written once every member has
          // passed this exchange (each wrote its columns, then fenced)
          ++s;
          const int tw = (int)threadIdx.x;
          if (!exchange_row(p, xb, s, tw < CLv, c_lo + min(tw, CLv - 1), 0.0f, row, sflag)) F = __builtin_nan("");
          __threadfence();
        }
      }
      if (lead && threadIdx.x == 0) p.offs[(size_t)item] = F;
    }
    __syncthreads();
    if (lead) {
      if (FWD) {
        finish_partition<CH::kLog>(p, b, len, F, n_re);
      } else if (threadIdx.x == 0 && p.recomputed != nullptr) {
        p.recomputed[b] = n_re;
      }
      // a group that gave up leaves NaN results: mark the sequence for the caller
      if (threadIdx.x == 0 && p.recomputed != nullptr && aborted(p)) p.recomputed[b] = -1;
    }
    __syncthreads();
  }
}

// Fills the exchange buffer with zero stamps and clears the abort flag.
__global__ void coop_clear_kernel(unsigned long long* xch, size_t n, int* xabort, int clear_abort) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    xch[i] = 0ull;
  if (clear_abort && blockIdx.x == 0 && threadIdx.x == 0) *xabort = 0;
}

// Clears the exchange buffer (and, first in a direction, the abort flag), then
// launches `kernel` cooperatively over all groups.
template <class K>
hipError_t launch_coop(K kernel, const Plan& pl, const ScanParams& p, int clear_abort, hipStream_t st) {
  const size_t n = (size_t)p.NQ * 2 * p.C;
  hipLaunchKernelGGL(coop_clear_kernel, dim3((unsigned)std::min<size_t>((n + 255) / 256, 1024)), dim3(256), 0, st,
                     p.xch, n, p.xabort, clear_abort);
  ScanParams q = p;
  void* args[] = {&q};
  return hipLaunchCooperativeKernel((const void*)kernel, dim3(pl.CGRID), dim3(pl.CNT), args, (unsigned)pl.coop_lds,
                                    st);
}

// One direction: main pass, verification, retry, verification, repair, offsets.
template <class CH>
int launch_coop_dir(const Plan& pl, const ScanParams& p, hipStream_t st) {
  constexpr bool fwd = CH::kFwd;
  auto k = coop_scan_kernel<CH>;
  auto kr = coop_retry_kernel<CH>;
  auto kf = coop_fixup_kernel<CH>;
  for (const void* f : {(const void*)k, (const void*)kr, (const void*)kf}) {
    hipError_t e = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl.coop_lds);
    if (e != hipSuccess) return e;
  }
  hipError_t e;
  {
    TimedLaunch tl(fwd ? kKScanFwd : kKScanBwd, st);
    e = launch_coop(k, pl, p, 1, st);
  }
  if (e != hipSuccess) return e;
  e = (hipError_t)launch_verify(pl, p, fwd, st);
  if (e != hipSuccess) return e;
  if (pl.P > 1) {
    {
      TimedLaunch tl(kKRetry, st);
      e = launch_coop(kr, pl, retry_params(p), 0, st);
    }
    if (e != hipSuccess) return e;
    e = (hipError_t)launch_verify(pl, p, fwd, st, true);
    if (e != hipSuccess) return e;
  }
  {
    TimedLaunch tl(fwd ? kKFwdFixup : kKBwdFixup, st);
    e = launch_coop(kf, pl, p, 0, st);
  }
  if (e != hipSuccess) return e;
  e = (hipError_t)launch_apply_offsets(pl, p, fwd, st);
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

}  // namespace coop
}  // namespace tsm
