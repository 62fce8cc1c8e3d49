// Register-resident log-semiring scan (forward alpha / backward beta) for gfx950.
//
// Same recursion, chunking and verification as the generic scan, with a data
// layout that makes one duration term cost one 8-byte LDS read, four VALU
// operations and one exponential:
//
//   * a group of J lanes serves one label c; lane j owns durations
//     k = 1 + j + J*r, r < R, with R a compile-time constant (padded
//     durations are masked through the duration bias register);
//   * the ring of label c holds, per position s, one fp64 value
//       x[s] = lvl[s] + v[s] - sgn*cum[s,c]*log2(e)
//     in a linear buffer of RL > KP entries: each step's position sits one index
//     below the previous one, so a step's KP reads are contiguous, and when the
//     index would drop below 0 the group copies its KP newest entries to the top
//     (once every RL - KP steps) -- half the LDS of a mirrored ring, so more
//     chunks share a CU;
//     (v = normalised state plus the projection a segment starting / ending at
//     s contributes, lvl = the position's fp64 level), so the term of duration
//     k at step t is x[s] + db[k] + sgn*cum[t,c]*log2(e) with s = t -/+ k;
//   * a lane sums its terms in one pass relative to its first term y0,
//     exp2((float)((x + db) - y0)) -- the large parts cancel in fp64 and only
//     the small exponent is rounded to fp32 (exact fallback to a two-pass
//     maximum when the sum overflows) -- then the J lanes combine;
//   * the ring of label c is read and written only by c's lane group, which
//     lives in one wavefront, so the only cross-wave exchange per step is the
//     row of all labels' results: one LDS barrier per step.
//
// sgn = +1 forward (content cum[t]-cum[t-k]), -1 backward (cum[t+k]-cum[t]).
//
// Emission input (EMIT, for p.emit != null): the chunk reads the projected scores
// (B, T, C) instead of cumulative scores and carries cum itself, in fp64, in a
// frame of its own: cum = 0 at its first position t_start, a running sum of
// the score rows stepped over after it, and prefix sums over the score rows
// behind a position for the ring entries there (behind_em).  The recursion
// only uses differences of cum along one label, so the frame drops out of every
// output; the emission prologue is fused into the scan's streamed loads and no
// (B, T+1, C) cumulative tensor is built.
//
// MARG (backward, log semiring, 16-lane groups): the beta scan also produces the
// segment marginals of the starts it owns.  The pull's term r of label c at
// step t is 2^(x[t+k] + db[k] - y0); times F = 2^(y0 + A[t,c]), with A the
// forward side of a segment starting at t (alpha level + u[t,c] + proj_start
// - cum[t,c] - log2 Z), it is P(t,k,c).  So each term costs three more
// multiplies/adds: the duration sums D[k,c] (per-lane registers), and the end
// sums E[t+k,c] (per-lane registers that slide one lane up the 16-lane DPP row
// each step, fused into the add).  The start sum S[t,c] comes from the pull's
// own log-sum.  Marginals are accumulated in the chunk's frame (see run()).
#pragma once

#include <float.h>

#include "tsm_chunk_driver.hpp"

namespace tsm {
namespace fastscan {

using namespace scan_detail;

constexpr double kInvD = -1e30;  // ring value of a position that does not exist
constexpr double kLog2eD = 1.4426950408889634;

// Wait for this wave's LDS operations, then barrier.  Global loads in flight
// (next-step prefetches) stay in flight.
__device__ __forceinline__ void lds_barrier() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// Compiler-only ordering point between a wave's LDS writes and its later reads
// of the same words by other lanes (LDS executes a wave's operations in order).
__device__ __forceinline__ void wave_lds_order() { __asm__ volatile("" ::: "memory"); }

// IN: the kind of problem a compiled instance serves -- kInCum (cumulative
// scores), kInEmit (projected scores, see above) or kInWin (cumulative scores,
// the problem being one window of a longer sequence in the bounded-memory
// backward, see below).  Each is its own kernel, so the plain instances carry
// none of the other kinds' code.
constexpr int kInCum = 0, kInEmit = 1, kInWin = 2;

template <int J, int R, bool FWD, bool LOGSR, bool MARG = false, int CJ = 4, int IN = kInCum>
struct Chunk {
  static constexpr bool EMIT = IN == kInEmit;
  // Window of a longer sequence (bounded-memory backward): chunks that would
  // start exactly from the sequence start (forward) or end (backward) start
  // from the state the caller hands over instead (p.org_st / p.org_lv, per
  // sequence, where p.org_ok[b] is set), in the ring format the chunks record
  // (positions 0, -1, ... forward; len, len+1, ... backward; global levels).
  // The forward can also record alpha-hat rows at multiples of p.ck_every
  // (p.ck_ah / p.ck_al).  The fused backward's top chunk then is exact in the
  // global frame (frame factor 1), sends the end sums of positions beyond len
  // to p.thalo, and chunk 0 records its boundary state at position 0 in
  // p.tst_st / p.tst_lv for the window below.
  static constexpr bool WIN = IN == kInWin;
  // Fused marginals: where the end sums E[s,c] (the probability that a segment
  // of label c ends at s) come from.  The cumulative-score instance takes them
  // at each owned step s from the tables themselves, E = 2^(alpha[s,c] +
  // beta[s,c] - log2 Z) (alpha from the forward's table, beta the step's own
  // mixed state), one exponential per (s, c).  The emission and window
  // instances slide per-term end sums along a DPP row instead (three more
  // operations per term): with emission input the score gradient is a running
  // sum of E - S over all later positions, which needs E and S summed from the
  // same terms, and a window's top chunk hands the end sums of segments that
  // cross into the window above to that window.
  static constexpr bool ESLIDE = EMIT || WIN;
  static_assert(!MARG || (!FWD && LOGSR && J == 16), "fused marginals: backward log scan, 16-lane DPP rows");
  static constexpr int kCJ = CJ;
  static constexpr bool kFwd = FWD;
  static constexpr bool kLog = LOGSR;
  static constexpr int kMaxThreads = R > 16 ? 512 : 1024;
  __device__ static double* red(char* smem, const ScanParams& p) {
    return reinterpret_cast<double*>(smem + fast_lds_layout(p.C, p.RL, p.RS, 0).red);
  }
  // Emission input: sgn * cum * log2(e), in the chunk's frame, of the position i
  // behind `base` (FWD: base - i, BWD: base + i), for i = i0 + lj of one block of
  // J consecutive i.  `carry` holds the value of position i0 - 1 (of base itself
  // when i0 == 0, where lane 0 adds nothing) and advances to i0 + J - 1.
  // Stepping back over a position lowers the value by that position's score row
  // times log2(e) in both directions.  Rows outside [0, T) are clamped: the
  // positions they lead to lie outside the sequence and are never used.  Every
  // lane of the J-lane group takes part (shuffles within the group).
  __device__ static double behind_em(const float* em_b, int C, int c, int T, int lj, int base, int i,
                                     double& carry) {
    double d = 0.0;
    if (i >= 1) {
      int row = FWD ? base - i : base + i - 1;
      row = row < 0 ? 0 : (row > T - 1 ? T - 1 : row);
      d = (double)em_b[(size_t)row * C + c];
    }
#pragma unroll
    for (int o = 1; o < J; o <<= 1) {
      const double v = __shfl_up(d, o, J);
      if (lj >= o) d += v;
    }
    const double val = carry - d * kLog2eD;
    carry = __shfl(val, J - 1, J);
    return val;
  }
  // ---------------------------------------------------------------------------
  // One chunk of one sequence.
  //   FWD: mode 0 exact from position 0; 1 speculative from t_lo - W; 2 exact
  //        from (init_st, init_lv) at t_lo.  Steps t = t_start+1 .. t_hi.
  //   BWD: mode 0 exact from position len; 1 speculative from t_hi + W; 2 exact
  //        from the state at t_hi.  Steps t = t_start-1 .. t_lo.
  // ---------------------------------------------------------------------------
  __device__ static void run(const ScanParams& p, char* smem, int b, int j, int mode, const float* init_st,
                             const double* init_lv) {
    constexpr int KP = J * R;
    const int C = p.C, Kmax = p.Kmax, K = p.K, RS = p.RS, RL = p.RL, T = p.T;
    const int len = seq_len(p, b);
    const int item = b * p.P + j;
    const FastLds L = fast_lds_layout(C, RL, RS, 0);
    double* ring = reinterpret_cast<double*>(smem + L.ring);
    double* lring = reinterpret_cast<double*>(smem + L.lring);
    float* row = reinterpret_cast<float*>(smem + L.row);
    const int tid = threadIdx.x, NT = blockDim.x;
    const int g = tid / J, lj = tid % J;
    const bool cval = g < C;
    const int c = cval ? g : C - 1;  // padding groups shadow the last label and never write
    constexpr bool emit = EMIT;
    // window: a chunk that starts from the handed-over state
    [[maybe_unused]] const bool from_org = WIN && mode == 0 && p.org_st != nullptr && p.org_ok[b] != 0;
    if constexpr (WIN) {
      if (from_org) {
        init_st = p.org_st + (size_t)b * Kmax * C;
        init_lv = p.org_lv + (size_t)b * Kmax;
      }
    }
    // (a window's inputs are rows of the full tensors: their sequence strides)
    const size_t xseq = WIN ? (size_t)p.xseq : (size_t)(T + 1) * C;
    const size_t pseq = WIN ? (size_t)p.pseq : (size_t)T * C;
    const float* cum_b = p.cum + (size_t)b * xseq;  // not read with emission input
    const float* em_b = emit ? p.emit + (size_t)b * T * C : nullptr;
    const bool has_ps = p.ps != nullptr, has_pe = p.pe != nullptr;
    const float* ps_b = has_ps ? p.ps + (size_t)b * pseq : nullptr;
    const float* pe_b = has_pe ? p.pe + (size_t)b * pseq : nullptr;
    const bool store = !MARG && p.val != nullptr;  // the fused backward keeps no beta table
    const double sgn = FWD ? 1.0 : -1.0;
    // fp64 cumulative score of position pos (own label) in log2 units, times sgn
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
    // duration bias in log2 units: fp32 products, widened to fp64 where they are used
    float dbr[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int k = 1 + lj + J * r;
      const int di = k < K - 1 ? k : K - 1;
      dbr[r] = (k <= Kmax) ? p.db[(size_t)di * C + c] * kLog2e : (float)kInvD;
    }
    // Kmax = 1: the duration-1 bias of the label (the register-0 bias of lane 0)
    [[maybe_unused]] const bool k1 = Kmax == 1;
    [[maybe_unused]] const float db1 = p.db[(size_t)(K > 1 ? 1 : 0) * C + c] * kLog2e;
    float trr[kCJ];
#pragma unroll
    for (int i = 0; i < kCJ; ++i) {
      const int ci = lj + J * i;
      // forward mix: own label c is the destination, ci the source; backward: c is the source
      trr[i] = (ci < C) ? (FWD ? p.trans[(size_t)ci * C + c] : p.trans[(size_t)c * C + ci]) * kLog2e : 0.0f;
    }
    // duration-bias factors relative to the lane's first duration: the pull's term r
    // is 2^(e[r] - e[0]) * edb[r] = 2^((e[r] + dbr[r]) - (e[0] + dbr[0])), one fp64
    // subtraction, conversion, exponential and FMA.  Padded durations get 0.  A lane
    // whose factors span more than 2^64 (an underflowed 2^(e[r]-e[0]) could then
    // still matter) always takes the exact two-pass path.
    float edb[R];
    bool lane_exact = false;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const double d = (double)dbr[r] - (double)dbr[0];
      edb[r] = exp2_hw((float)d);
      // (fused marginals without sliding end sums also divide by the factor: keep it >= 2^-64)
      lane_exact = lane_exact || (d > 64.0) || (MARG && !ESLIDE && d < -64.0 && 1 + lj + J * r <= Kmax);
    }

    // ---- empty rings ----
    for (int idx = tid; idx < C * RL; idx += NT) ring[idx] = kInvD;
    for (int i = tid; i < RS; i += NT) lring[i] = 0.0;
    __syncthreads();

    double* rc = ring + (size_t)c * RL;
    // position t_start at index A0, the positions behind it at A0 + i
    const int A0 = RL - KP;
    double lvl_prev;

    // ---- fused marginals (MARG) ----
    // The chunk's beta values carry a frame offset d (its levels are the exact
    // ones minus offs[item], known only after verification).  At its first
    // owned start, t_hi - 1, the chunk takes the largest alpha*beta/Z of the
    // positions t_hi .. t_hi+Kmax-1 in its own frame, 2^fr.  Every segmentation
    // has a boundary among any Kmax consecutive positions, so the true value is
    // >= 1/(Kmax*C) and d - fr lies in [0, log2(Kmax*C)]: marginals accumulate
    // as P * 2^(d - fr) without fp32 overflow, and the finalize multiplies them
    // by 2^(fr + offs[item]).  zd = log2 Z + fr.
    [[maybe_unused]] const float* u_b = MARG ? p.uval + (size_t)b * (T + 1) * C : nullptr;
    [[maybe_unused]] const double* al_b = MARG ? p.alvl + (size_t)b * (T + 1) : nullptr;
    [[maybe_unused]] float* e_own_b = MARG ? p.e_own + (size_t)b * (T + 1) * C : nullptr;
    [[maybe_unused]] float* s_out_b = MARG ? p.s_out + (size_t)b * (T + 1) * C : nullptr;
    [[maybe_unused]] float* halo_i = MARG ? p.halo + (size_t)item * Kmax * C : nullptr;
    [[maybe_unused]] const int own_hi = (FWD || j < jl) ? t_hi : len + 1;  // rows [t_lo, own_hi) are this chunk's
    [[maybe_unused]] const int lane_last = (lj == J - 1) ? -1 : 0;       // all bits set on the row's last lane
    // Duration sums: fp32 per lane, added every 128 owned steps (each (k, c) has
    // one lane; an fp32 sum of at most 128 positive terms is within 128 ulp) to
    // fp64 sums.  Up to 20 durations per lane those are registers, written to
    // the chunk's partials once at the end: the kernel runs one workgroup per CU
    // (its rings fill the LDS), so the 2R extra registers cost no occupancy,
    // where the periodic 8-byte atomics they replace wrote about 0.5 GB per
    // launch at cfg3.  Longer lanes (no room in 256 registers) add into the
    // zeroed partials with no-return atomics, which never contend.
    constexpr bool kRegD = R <= 20;
    double zd = 0.0;
    float d32[MARG ? R : 1], ea[(MARG && ESLIDE) ? R : 1];
    double d64[MARG && kRegD ? R : 1];
    [[maybe_unused]] double* dbp = MARG ? p.db_part + (size_t)item * Kmax * C : nullptr;
    if constexpr (MARG) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        d32[r] = 0.0f;
        if constexpr (ESLIDE) ea[r] = 0.0f;
        if constexpr (kRegD) {
          d64[r] = 0.0;
        } else {
          const int k = 1 + lj + J * r;
          if (cval && k <= Kmax) dbp[(size_t)(k - 1) * C + c] = 0.0;
        }
      }
      if (tid == 0) p.mframe[item] = 0.0;
      if constexpr (!kRegD) __threadfence();  // the zeros before the first atomic add
    }
    // (without sliding end sums the fp32 sums hold x * F: times the register's
    // duration-bias factor, or 1 on a lane with extreme factors, when folded)
    auto fold_d = [&]() {
      if constexpr (MARG && kRegD) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          d64[r] += (double)((ESLIDE || lane_exact) ? d32[r] : d32[r] * edb[r]);
          d32[r] = 0.0f;
        }
      } else if constexpr (MARG) {
        // addresses and masks from an opaque copy of the lane index: otherwise they
        // are hoisted out of the step loop and held in registers throughout
        int ljo = lj;
        __asm__ volatile("" : "+v"(ljo));
        double* a = dbp + (size_t)ljo * C + c;
#pragma unroll
        for (int r = 0; r < R; ++r) {
          if (cval && 1 + ljo + J * r <= Kmax)
            unsafeAtomicAdd(a, (double)((ESLIDE || lane_exact) ? d32[r] : d32[r] * edb[r]));
          a += (size_t)J * C;
          d32[r] = 0.0f;
        }
      }
    };
    // ---- initial state ----
    if (mode == 0 && !from_org) {
      const int pos = t_start;  // FWD: 0, BWD: len
      lvl_prev = 0.0;
      float v0;
      if (FWD) {
        // alpha-hat[0] = 0 for every label; u[0,c] = (+)_{c'} trans[c',c]
        float m = kMinusInf;
        int mi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < kCJ; ++i)
          if (lj + J * i < C && trr[i] > m) {
            m = trr[i];
            mi = lj + J * i;
          }
        float u0;
        if constexpr (LOGSR) {
          float sm = 0.0f;
#pragma unroll
          for (int i = 0; i < kCJ; ++i)
            if (lj + J * i < C) sm += exp2_hw(trr[i] - m);
          u0 = group_lse2<J>(m, sm);
        } else {
          // Viterbi: best source label of a segment starting at position 0
          const ValIdx best = group_argmax_first<J>(ValIdx{m, mi});
          u0 = best.v;
          if (p.bp != nullptr && cval && lj == 0 && j == 0) p.bp[((size_t)b * (T + 1)) * C + c] = best.i;
        }
        v0 = u0 + ((has_ps && T > 0) ? ps_b[c] * kLog2e : 0.0f);
        if (g == 0) {
#pragma unroll
          for (int i = 0; i < kCJ; ++i) {
            const int ci = lj + J * i;
            if (ci < C) {
              if (store && j == 0) p.val[((size_t)b * (T + 1)) * C + ci] = 0.0f;
              if (len == 0) p.fin[(size_t)b * C + ci] = 0.0f;
            }
          }
        }
        if (tid == 0) {
          if (store && j == 0) p.lvl[(size_t)b * (T + 1)] = 0.0;
          if (len == 0) p.fin_lvl[b] = 0.0;
        }
      } else {
        v0 = (has_pe && len >= 1) ? pe_b[(size_t)(len - 1) * C + c] * kLog2e : 0.0f;
        if (cval && lj == 0 && store) p.val[((size_t)b * (T + 1) + len) * C + c] = 0.0f;
        if (tid == 0 && store) p.lvl[(size_t)b * (T + 1) + len] = 0.0;
      }
      if (cval && lj == 0) rc[A0] = (double)v0 - (emit ? 0.0 : cumx(pos));
      if (tid == 0) lring[pos % RS] = 0.0;
    } else {
      lvl_prev = (mode == 1) ? 0.0 : init_lv[0];
      // positions t_start -/+ i, i < Kmax
      if constexpr (EMIT) {
        if (cval) {
          double carry = 0.0;  // the chunk's frame has cum = 0 at t_start
          for (int i0 = 0; i0 < Kmax; i0 += J) {
            const int i = i0 + lj;
            const double cxp = behind_em(em_b, C, c, T, lj, t_start, i, carry);
            if (i >= Kmax) continue;
            const int pos = FWD ? t_start - i : t_start + i;
            float v;
            if (mode == 1) {
              if (FWD) v = has_ps ? ps_b[(size_t)pos * C + c] * kLog2e : 0.0f;
              else v = has_pe ? pe_b[(size_t)(pos - 1) * C + c] * kLog2e : 0.0f;
            } else {
              v = init_st[(size_t)i * C + c];
            }
            const double lv = (mode == 1) ? 0.0 : init_lv[i];
            rc[A0 + i] = lv + (double)v - cxp;
          }
        }
      } else if constexpr (WIN) {
        // as below; positions before the window (forward) or beyond the sequence
        // (backward) may be involved: entries marked "does not exist" read no
        // cumulative score, and level slots wrap for negative positions
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
            // (forward: pos may be negative, a position of the window below)
            rc[A0 + i] = (v < -1e29f) ? kInvD : lv + (double)v - sgn * (double)cum_b[(ptrdiff_t)pos * C + c] * kLog2eD;
          }
        }
      } else {
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
      }
      for (int i = tid; i < Kmax; i += NT) {
        const int pos = FWD ? t_start - i : t_start + i;
        if constexpr (WIN) lring[((pos % RS) + RS) % RS] = (mode == 1) ? 0.0 : init_lv[i];
        else lring[pos % RS] = (mode == 1) ? 0.0 : init_lv[i];
      }
    }
    __syncthreads();

    // ---- per-step operands ----
    const int dir = FWD ? 1 : -1;
    const int t_first = t_start + dir;
    const int t_end = FWD ? t_hi + 1 : t_lo - 1;  // exclusive
    auto clampT = [&](int t) { return t < 0 ? 0 : (t > T ? T : t); };
    auto clampT1 = [&](int t) { return t < 0 ? 0 : (t > T - 1 ? T - 1 : t); };
    // projection operands: forward adds proj_end[t-1] to the pull and proj_start[t]
    // to the ring entry; backward adds proj_start[t] to the pull and proj_end[t-1]
    // to the ring entry.  Absent projections are not read (operand 0, scale 0).
    // per step: cum[t] (cum input) or the score row stepped over, t-1 forward and t
    // backward (emission input), whose running sum is the chunk-frame cum
    const float* xs_b = emit ? em_b : cum_b;
    auto xs_row = [&](int t) { return emit ? clampT1(FWD ? t - 1 : t) : clampT(t); };
    const float* pa_src = FWD ? (has_pe ? pe_b : xs_b) : (has_ps ? ps_b : xs_b);
    const float* pb_src = FWD ? (has_ps ? ps_b : xs_b) : (has_pe ? pe_b : xs_b);
    const float pa_scale = (FWD ? has_pe : has_ps) ? kLog2e : 0.0f;
    const float pb_scale = (FWD ? has_ps : has_pe) ? kLog2e : 0.0f;
    const bool has_pa = FWD ? has_pe : has_ps, has_pb = FWD ? has_ps : has_pe;
    auto pa_row = [&](int t) { return FWD ? clampT1(t - 1) : clampT1(t); };
    auto pb_row = [&](int t) { return FWD ? clampT1(t) : clampT1(t - 1); };
    // emission input: the running sgn * cum * log2(e) of the previous position
    [[maybe_unused]] double cx_run = 0.0;
    [[maybe_unused]] const float* ah_b = MARG ? p.aval + (size_t)b * (T + 1) * C : nullptr;
    // Scans without marginals: the operands of the next step, loaded one step ahead.
    [[maybe_unused]] float cum_n = 0.0f, pa_n = 0.0f, pb_n = 0.0f;
    // Fused marginals (six operands per step): the operands of step si (si = 0, 1, ...
    // from t_first) go through LDS in batches of SB <= J steps (SB = p.SB, a power of
    // two).  Lane lj < SB of a group loads those of step n*SB + lj of batch n one
    // batch early and writes them to the group's slots at the first step of batch n,
    // when every read of batch n-1's slots is done (a wave runs its LDS operations in
    // order), so a global load has SB steps to arrive instead of one.  Slots: two
    // float4 per step (score row, proj_end side, proj_start side, u; alpha-hat row and
    // the fp64 alpha level), and one float4 of padding per group so that the groups
    // of a wave read different banks.
    [[maybe_unused]] const int SB = MARG ? p.SB : 1;
    [[maybe_unused]] const int sbs = __builtin_ctz((unsigned)SB);
    [[maybe_unused]] float4* stg = reinterpret_cast<float4*>(smem + L.stage) + (size_t)g * (2 * SB + 1);
    [[maybe_unused]] float qx = 0.0f, qa = 0.0f, qb = 0.0f, qu = 0.0f, qh = 0.0f;
    [[maybe_unused]] double ql = 0.0;
    [[maybe_unused]] auto stage_load = [&](int n) {
      const int tq = t_first + dir * (n * SB + lj);
      qx = xs_b[(size_t)xs_row(tq) * C + c];
      qa = has_pa ? pa_src[(size_t)pa_row(tq) * C + c] : 0.0f;
      qb = has_pb ? pb_src[(size_t)pb_row(tq) * C + c] : 0.0f;
      qu = u_b[(size_t)clampT(tq) * C + c];
      ql = al_b[clampT(tq)];
      if constexpr (!ESLIDE) qh = ah_b[(size_t)clampT(tq) * C + c];
    };
    if constexpr (MARG) {
      stage_load(0);
    } else {
      cum_n = xs_b[(size_t)xs_row(t_first) * C + c];
      pa_n = has_pa ? pa_src[(size_t)pa_row(t_first) * C + c] : 0.0f;
      pb_n = has_pb ? pb_src[(size_t)pb_row(t_first) * C + c] : 0.0f;
    }

    const int rec_spec = (mode == 1) ? (FWD ? t_lo : t_hi) : -1;
    // (window: the backward's chunk 0 records its state at position 0 for the window below)
    const int rec_end = FWD ? ((t_hi < len) ? t_hi : -1)
                            : ((j >= 1 || (WIN && p.tst_st != nullptr)) ? t_lo : -1);

    int A = A0;  // ring index of the current position
    // single duration: the ring entry of the previous position (the only one a step
    // reads) also kept in a register; every lane of the label group computes it
    [[maybe_unused]] double xr = (!MARG && R == 1 && k1) ? rc[A0] : 0.0;
    // per-step offsets kept as running values (uniform): row t of the (B, T+1, C) tables,
    // entry t of the (B, T+1) levels, row t of this sequence's tables, and t mod RS
    size_t row_off = ((size_t)b * (T + 1) + t_first) * C;
    size_t lvl_off = (size_t)b * (T + 1) + t_first;
    [[maybe_unused]] size_t tc_off = (size_t)t_first * C;
    int lr = ((t_first % RS) + RS) % RS;
    for (int t = t_first; t != t_end; t += dir) {
      if constexpr (MARG) {
        if (WIN && from_org && t == t_hi - 1) {
          // window: a chunk that starts from the handed-over state is exact in the
          // global frame, so its marginals need no frame (factor 1)
          zd = p.mz2[b];
          if (tid == 0) p.mframe[item] = 0.0;
        } else if (t == t_hi - 1) {
          // frame estimate from the ring of position t_hi (index A) and the Kmax-1 behind
          // it; operands from an opaque copy of the sequence index, so that nothing of
          // this once-per-chunk block is hoisted out of the step loop
          int bo = b;
          __asm__ volatile("" : "+s"(bo));
          const size_t row0 = (size_t)bo * (T + 1);
          double m = -1e300;
          if constexpr (EMIT) {
            if (cval) {
              double carry = cx_run;  // position t_hi (the previous step, or t_start)
              for (int i0 = 0; i0 < Kmax; i0 += J) {
                const int i = i0 + lj;
                const double cxv = behind_em(em_b, C, c, T, lj, t_hi, i, carry);
                const int pos = t_hi + i;
                if (i < Kmax && pos <= len) {
                  const double pbv = (has_pe && pos >= 1) ? (double)(p.pe[((size_t)bo * T + pos - 1) * C + c] * kLog2e) : 0.0;
                  const double lb = (rc[A + i] - pbv) + cxv;  // log2 beta(pos, c), chunk frame
                  const double la = (double)p.aval[(row0 + pos) * C + c] + p.alvl[row0 + pos];
                  m = fmax(m, la + lb);
                }
              }
            }
          } else {
            if (cval) {
              for (int i = lj; i < Kmax; i += J) {
                const int pos = t_hi + i;
                if (pos <= len) {
                  const double pbv =
                      (has_pe && pos >= 1)
                          ? (double)((WIN ? pe_b[(size_t)(pos - 1) * C + c] : p.pe[((size_t)bo * T + pos - 1) * C + c]) *
                                     kLog2e)
                          : 0.0;
                  const double cxv = -(double)(WIN ? cum_b[(size_t)pos * C + c] : p.cum[(row0 + pos) * C + c]) * kLog2eD;
                  const double lb = (rc[A + i] - pbv) + cxv;  // log2 beta(pos, c), chunk frame
                  const double la = (double)p.aval[(row0 + pos) * C + c] + p.alvl[row0 + pos];
                  m = fmax(m, la + lb);
                }
              }
            }
          }
          double mn;
          block_minmax(m, m, red(smem, p), zd, mn);
          if (tid == 0) p.mframe[(size_t)bo * p.P + j] = zd - p.mz2[bo];
          if constexpr (!ESLIDE) {
            // the last chunk also owns row len, the start state of the scan (beta
            // level 0, no label mix): E[len] = 2^(alpha[len] - log2 Z)
            if (j == jl && cval && lj == 0)
              e_own_b[(size_t)len * C + c] =
                  exp2_hw((float)(p.alvl[row0 + len] - zd) + p.aval[(row0 + len) * C + c]);
          }
        }
      }
      if (--A < 0) {
        // the KP newest entries (indices 0 .. KP-1) to the top; each label group
        // copies its own ring inside its wavefront (LDS keeps a wave's order)
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
      // ---- this step's operands ----
      float x_t, pa_v, pb_v;
      [[maybe_unused]] float u_t = 0.0f, ah_t = 0.0f;
      [[maybe_unused]] double la_t = 0.0;
      if constexpr (MARG) {
        // slot si mod SB of the staged batch
        const int si = (t - t_first) * dir;
        const int slot = si & (SB - 1);
        if (slot == 0) {
          if (lj < SB) {
            stg[2 * lj] = make_float4(qx, qa, qb, qu);
            stg[2 * lj + 1] = make_float4(qh, __int_as_float(__double2loint(ql)), __int_as_float(__double2hiint(ql)), 0.0f);
          }
          wave_lds_order();
          stage_load((si >> sbs) + 1);
        }
        const float4 o0 = stg[2 * slot];
        const float4 o1 = stg[2 * slot + 1];
        x_t = o0.x;
        pa_v = o0.y;
        pb_v = o0.z;
        u_t = o0.w;
        ah_t = o1.x;
        la_t = __hiloint2double(__float_as_int(o1.z), __float_as_int(o1.y));
      } else {
        x_t = cum_n;
        pa_v = pa_n;
        pb_v = pb_n;
        const int tn = t + dir;
        cum_n = xs_b[(size_t)xs_row(tn) * C + c];
        if (has_pa) pa_n = pa_src[(size_t)pa_row(tn) * C + c];
        if (has_pb) pb_n = pb_src[(size_t)pb_row(tn) * C + c];
      }
      double cx_t;
      if constexpr (EMIT) cx_t = cx_run = cx_run + (double)x_t * kLog2eD;
      else cx_t = sgn * (double)x_t * kLog2eD;
      const float pa_t = pa_v * ((FWD ? t >= 1 : true) ? pa_scale : 0.0f);
      const float pb_t = pb_v * ((FWD ? true : t >= 1) ? pb_scale : 0.0f);

      // ---- pull over the lane's durations ----
      const double* rb = rc + A + 1 + lj;
      double e[R];
      if (!(!MARG && R == 1 && k1)) {
#pragma unroll
        for (int r = 0; r < R; ++r) e[r] = rb[J * r];
      }
      float a2;
      int kbest = 0;
      if (!MARG && R == 1 && k1) {
        // a single duration (Kmax = 1, the HMM): the term of lane 0 (ring entry of the
        // previous position, xr), which every lane computes itself; the group
        // reduction would return exactly this value
        a2 = (float)(((xr + (double)db1) + cx_t) - lvl_prev) + pa_t;
        kbest = 1;
      } else if constexpr (LOGSR) {
        double y0 = e[0] + (double)dbr[0];
        float s0 = 1.0f, s1 = 0.0f;
        // MARG: the lane's terms 2^(x + db - y0); without sliding end sums, the
        // terms without their duration-bias factor (D sums x * F, and the fold
        // multiplies by the factor, which is constant per register)
        float tm[MARG ? R : 1];
        if constexpr (MARG) tm[0] = 1.0f;
#pragma unroll
        for (int r = 1; r < R; ++r) {
          const float x = exp2_hw((float)(e[r] - e[0]));
          if constexpr (MARG && ESLIDE) {
            tm[r] = x * edb[r];
            if (r & 1) s1 += tm[r];
            else s0 += tm[r];
          } else if constexpr (MARG) {
            tm[r] = x;
            if (r & 1) s1 = fmaf(x, edb[r], s1);
            else s0 = fmaf(x, edb[r], s0);
          } else {
            if (r & 1) s1 = fmaf(x, edb[r], s1);
            else s0 = fmaf(x, edb[r], s0);
          }
        }
        float s = s0 + s1;
        // overflow (inf, or inf * 0 = NaN on a padded duration) or extreme factors
        if (__ballot(!(s <= FLT_MAX) || lane_exact)) {
          // a later term exceeds the first by more than the fp32 exponent range.
          // The fp64 biases are widened here from opaque copies: widened outside the
          // step loop they would hold 2R registers throughout.
          double ey[R];
#pragma unroll
          for (int r = 0; r < R; ++r) {
            float dv = dbr[r];
            __asm__ volatile("" : "+v"(dv));
            ey[r] = e[r] + (double)dv;
          }
          double m = y0;
#pragma unroll
          for (int r = 1; r < R; ++r) m = fmax(m, ey[r]);
          s = 0.0f;
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const float q = exp2_hw((float)(ey[r] - m));
            if constexpr (MARG && ESLIDE) {
              tm[r] = q;
            } else if constexpr (MARG) {
              // a lane with extreme factors keeps the whole term (its fold multiplies by 1)
              tm[r] = (lane_exact || !(edb[r] > 0.0f)) ? q : q * __builtin_amdgcn_rcpf(edb[r]);
            }
            s += q;
          }
          y0 = m;
        }
        // the lane's terms relative to the previous position's level
        const double yrel = (y0 + cx_t) - lvl_prev;
        [[maybe_unused]] double lam = 0.0;
        [[maybe_unused]] float sp = 0.0f;  // emission input: the lane's sum of P (start sum)
        if constexpr (MARG) {
          if (t < t_hi) {
            // P(t,k,c) = term * 2^(y0 + A[t,c]) in the chunk frame
            lam = (lvl_prev + la_t) - zd;
            const float yA = (float)(yrel + lam) + (u_t + pa_t);
            float F = exp2_hw(yA);
            if (__ballot(yA < -100.0f && s > 0x1p20f)) {
              // F underflows while later terms (<= FLT_MAX) are large enough to matter:
              // scale in two steps, 2^(yA+100) (no overflow) then 2^-100 (exact)
              const float F1 = exp2_hw(yA + 100.0f);
#pragma unroll
              for (int r = 0; r < R; ++r) tm[r] = (tm[r] * F1) * 0x1p-100f;
              F = 1.0f;
            }
            if constexpr (!ESLIDE) {
              // duration sums only (end sums from the tables, after the label mix)
#pragma unroll
              for (int r = 0; r < R; ++r) d32[r] += tm[r] * F;
            } else {
            // the end sum of position t+1+KP (lane J-1, register R-1) is complete: out
            const int pr = t + 1 + KP;
            if (cval && lj == J - 1 && pr <= t_hi - 1 + Kmax && pr <= len) {
              if (pr < own_hi) e_own_b[(size_t)pr * C + c] = ea[R - 1];
              else halo_i[(size_t)(pr - t_hi) * C + c] = ea[R - 1];
            }
            if constexpr (WIN) {
              // window: end sums beyond len (positions of the window above): the top
              // chunk's to thalo, the chunk below it keeps them in its halo rows
              if (p.thalo != nullptr && cval && lj == J - 1 && pr > len) {
                if (j == jl && from_org && pr <= len + Kmax - 1) p.thalo[((size_t)b * Kmax + (pr - len - 1)) * C + c] = ea[R - 1];
                else if (j < jl && pr <= t_hi - 1 + Kmax) halo_i[(size_t)(pr - t_hi) * C + c] = ea[R - 1];
              }
            }
            // end sums slide to positions t+1+lj+16r: the last lane takes the previous
            // register (register 0: the new position t+1), then the row rotates one
            // lane up, fused with the accumulation.  Descending r reads ea[r-1] first.
#pragma unroll
            for (int r = R - 1; r >= 0; --r) {
              const float P = tm[r] * F;
              d32[r] += P;
              if constexpr (EMIT) sp += P;
              const float prv = (r >= 1) ? ea[r - 1] : 0.0f;
              // a bitwise merge: a select would become a register-array read at a lane-dependent index
              const float sl = __int_as_float((__float_as_int(prv) & lane_last) | (__float_as_int(ea[r]) & ~lane_last));
              ea[r] = add_row_ror1(sl, P);
            }
            }
          }
        }
        // combined over the group
        a2 = group_lse2<J>((float)yrel, s) + pa_t;
        if constexpr (MARG) {
          if (t < t_hi) {
            // start sum: sum_k P = 2^(lvl_prev + a2 + alpha level + u - zd).  Emission
            // input: the sum of the same P terms the end sums take, so that the score
            // gradient, a running sum of E - S over all positions, carries no
            // relative bias between the two (the exp2 / log2 of the log-sum would
            // leave one of ~1e-7, which the running sum accumulates)
            if constexpr (EMIT) {
              const float St = group_sum<J>(sp);
              if (cval && lj == 0) s_out_b[tc_off + c] = St;
            } else {
              if (cval && lj == 0) s_out_b[tc_off + c] = exp2_hw((float)(lam + (double)a2) + u_t);
            }
            if (((t_hi - 1 - t) & 127) == 127) fold_d();
          }
        }
      } else {
        // max over durations; ties go to the smallest duration (lanes hold ascending k).
        // The fp64 biases are widened here from opaque copies (one conversion per
        // term): widened outside the step loop they would hold 2R registers.
        double ym = e[0] + (double)dbr[0];
        int km = 1 + lj;
#pragma unroll
        for (int r = 1; r < R; ++r) {
          float dv = dbr[r];
          __asm__ volatile("" : "+v"(dv));
          const double y = e[r] + (double)dv;
          if (y > ym) {
            ym = y;
            km = 1 + lj + J * r;
          }
        }
        const ValIdx best = group_argmax_first<J>(ValIdx{(float)((ym + cx_t) - lvl_prev), km});
        a2 = best.v + pa_t;
        kbest = best.i;
      }
      const int par = t & 1;
      if (cval && lj == 0) row[par * C + c] = a2;
      lds_barrier();

      // ---- all labels: normaliser and label mix ----
      float rv[kCJ];
      float ml = kMinusInf;
#pragma unroll
      for (int i = 0; i < kCJ; ++i) {
        const int ci = lj + J * i;
        rv[i] = (ci < C) ? row[par * C + ci] : kMinusInf;
        ml = fmax2(ml, rv[i]);
      }
      const float mx = group_max<J>(ml);
      const double lvl_t = lvl_prev + (double)mx;
      float mixv;
      if constexpr (LOGSR) {
        // the exponent shift of the mix is the source maximum of rv + trr, which
        // does not wait for the row maximum (the two group reductions overlap);
        // the shift only has to be near the largest term and is added back
        // exactly, the terms keep the form (rv - mx) + trr
        float mt = kMinusInf;
#pragma unroll
        for (int i = 0; i < kCJ; ++i)
          if (lj + J * i < C) mt = fmax2(mt, rv[i] + trr[i]);
        const float shift = group_max<J>(mt) - mx;
        float sq = 0.0f;
#pragma unroll
        for (int i = 0; i < kCJ; ++i)
          if (lj + J * i < C) sq += exp2_hw(((rv[i] - mx) + trr[i]) - shift);
        mixv = shift + log2_hw(group_sum<J>(sq));
      } else {
        float mq = kMinusInf;
        int mqi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < kCJ; ++i)
          if (lj + J * i < C) {
            const float q = (rv[i] - mx) + trr[i];
            if (q > mq) {
              mq = q;
              mqi = lj + J * i;
            }
          }
        // Viterbi: best source label for a segment starting at t (first on ties)
        const ValIdx best = group_argmax_first<J>(ValIdx{mq, mqi});
        mixv = best.v;
        if (FWD && p.bp != nullptr && cval && lj == 0 && (j == 0 || t > t_lo))
          p.bp[row_off + c] = (kbest << 16) | best.i;
      }

      const bool owned = FWD ? (j == 0 || t > t_lo) : (t < t_hi || j == jl);
      if (FWD) {
        if (g == 0) {
#pragma unroll
          for (int i = 0; i < kCJ; ++i) {
            const int ci = lj + J * i;
            if (ci < C) {
              const float ah = rv[i] - mx;
              if (store && owned) p.val[row_off + ci] = ah;
              if (t == len) p.fin[(size_t)b * C + ci] = ah;
              if constexpr (WIN) {
                // checkpoint rows of the bounded-memory backward (levels in the chunk frame)
                if (p.ck_ah != nullptr && owned && t % p.ck_every == 0 && t / p.ck_every < p.ck_n)
                  p.ck_ah[((size_t)(t / p.ck_every) * p.B + b) * C + ci] = ah;
              }
            }
          }
        }
        if (tid == 0) {
          if (store && owned) p.lvl[lvl_off] = lvl_t;
          if (t == len) p.fin_lvl[b] = lvl_t;
          if constexpr (WIN) {
            if (p.ck_ah != nullptr && owned && t % p.ck_every == 0 && t / p.ck_every < p.ck_n)
              p.ck_al[(size_t)(t / p.ck_every) * p.B + b] = lvl_t;
          }
        }
      } else {
        if (cval && lj == 0 && store && owned) p.val[row_off + c] = mixv;
        if (tid == 0 && store && owned) p.lvl[lvl_off] = lvl_t;
      }
      if constexpr (MARG && !ESLIDE) {
        // end sum of the owned row t: 2^(alpha[t,c] + beta[t,c] - log2 Z), beta the
        // mixed state of this step in the chunk frame; no segment ends at position 0
        if (t < t_hi && cval && lj == 0)
          e_own_b[tc_off + c] = (t == 0) ? 0.0f : exp2_hw((float)((la_t + lvl_t) - zd) + (ah_t + mixv));
      }
      // ---- ring entry for position t ----
      if (cval && lj == 0) {
        rc[A] = (lvl_t + (double)(mixv + pb_t)) - cx_t;
      }
      if (!MARG && R == 1 && k1) xr = (lvl_t + (double)(mixv + pb_t)) - cx_t;
      if (tid == 0) lring[lr] = lvl_t;
      lvl_prev = lvl_t;
      wave_lds_order();
      row_off += (ptrdiff_t)dir * C;
      lvl_off += dir;
      tc_off += (ptrdiff_t)dir * C;
      lr += dir;
      lr = (lr == RS) ? 0 : (lr < 0 ? RS - 1 : lr);

      // ---- boundary states for verification: positions t -/+ i, i < Kmax ----
      if (t == rec_spec || t == rec_end) {
        float* st = (t == rec_spec ? p.st_spec : p.st_end) + (size_t)item * Kmax * C;
        double* lv = (t == rec_spec ? p.lv_spec : p.lv_end) + (size_t)item * Kmax;
        if constexpr (WIN && !FWD) {
          if (t == rec_end && j == 0) {
            st = p.tst_st + (size_t)b * Kmax * C;
            lv = p.tst_lv + (size_t)b * Kmax;
          }
        }
        if constexpr (EMIT) {
          if (cval) {
            double carry = cx_t;
            for (int i0 = 0; i0 < Kmax; i0 += J) {
              const int i = i0 + lj;
              const double cxe = behind_em(em_b, C, c, T, lj, t, i, carry);
              if (i >= Kmax) continue;
              const int pos = FWD ? t - i : t + i;
              const double x = rc[A + i];
              const double lp = (i == 0) ? lvl_t : lring[pos % RS];
              // positions outside the sequence keep the "does not exist" marker
              st[(size_t)i * C + c] = (x < -1e29) ? -1e30f : (float)((x - lp) + cxe);
            }
          }
        } else {
          if (cval) {
            for (int i = lj; i < Kmax; i += J) {
              const int pos = FWD ? t - i : t + i;
              const double x = rc[A + i];
              const double lp = (i == 0) ? lvl_t : lring[pos % RS];
              // positions outside the sequence keep the "does not exist" marker
              st[(size_t)i * C + c] = (x < -1e29) ? -1e30f : (float)((x - lp) + cumx(pos));
            }
          }
        }
        if constexpr (WIN && !FWD) {
          // the state handed to the window below: there position 0 of this window is
          // the end of that window's sequence part, and its ring entry takes
          // proj_end of the row before it (segments ending there), which this
          // window's position 0 (no segment of the window ends there) leaves out
          if (t == rec_end && j == 0 && has_pe && cval && lj == 0) st[c] += pe_b[c - (ptrdiff_t)C] * kLog2e;
        }
        for (int i = tid; i < Kmax; i += NT) {
          const int pos = FWD ? t - i : t + i;
          lv[i] = (i == 0) ? lvl_t : lring[pos % RS];
        }
      }
    }
    if constexpr (MARG) {
      // rows still in the registers (lane lj, register r: position t_lo+1+lj+16r),
      // row t_lo (no own starts end there) and the duration sums
      if constexpr (ESLIDE) {
       if (cval) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
          const int pr = t_lo + 1 + lj + J * r;
          if (pr <= t_hi - 1 + Kmax && pr <= len) {
            if (pr < own_hi) e_own_b[(size_t)pr * C + c] = ea[r];
            else halo_i[(size_t)(pr - t_hi) * C + c] = ea[r];
          }
          if constexpr (WIN) {
            if (p.thalo != nullptr && pr > len) {
              if (j == jl && from_org && pr <= len + Kmax - 1) p.thalo[((size_t)b * Kmax + (pr - len - 1)) * C + c] = ea[r];
              else if (j < jl && pr <= t_hi - 1 + Kmax) halo_i[(size_t)(pr - t_hi) * C + c] = ea[r];
            }
          }
        }
        if (lj == 0) e_own_b[(size_t)t_lo * C + c] = 0.0f;
       }
      }
      fold_d();
      if constexpr (kRegD) {
        if (cval) {
#pragma unroll
          for (int r = 0; r < R; ++r) {
            const int k = 1 + lj + J * r;
            if (k <= Kmax) dbp[(size_t)(k - 1) * C + c] = d64[r];
          }
        }
      }
    }
  }
};

// source labels per lane of the label mix: 2 when C <= 2J, else 4 (the plan keeps C <= 4J);
// single-duration 8-lane plans with C <= 8 take 1 (launch_chunk_any)
template <int J>
inline bool narrow_mix(const ScanParams& p) { return p.C <= 2 * J; }

// The instance of one (direction, semiring, fusion): label-mix width from C,
// emission input from p.emit (each its own compiled kernel, so the cumulative-
// score instances carry none of the emission code's registers).
template <int J, int R, bool FWD, bool LOGSR, bool MARG>
int launch_chunk_any(const Plan& pl, const ScanParams& p, hipStream_t st) {
  if (p.win) {
    // windows of the bounded-memory backward: 16-lane log-semiring scans
    if constexpr (J == 16 && LOGSR && (FWD || MARG)) {
      if (p.emit != nullptr) return (int)hipErrorInvalidValue;
      return narrow_mix<J>(p) ? launch_chunk_dir<Chunk<J, R, FWD, LOGSR, MARG, 2, kInWin>>(pl, p, pl.fast_lds, pl.FNT, st)
                              : launch_chunk_dir<Chunk<J, R, FWD, LOGSR, MARG, 4, kInWin>>(pl, p, pl.fast_lds, pl.FNT, st);
    }
    return (int)hipErrorInvalidValue;
  }
  const bool em = p.emit != nullptr;
  if constexpr (J == 8 && R == 1 && !MARG) {
    // single-duration plans with no more labels than lanes per group (the HMM with
    // C <= 8): one source label per lane in the label mix
    if (!em && p.C <= J) return launch_chunk_dir<Chunk<J, R, FWD, LOGSR, MARG, 1, kInCum>>(pl, p, pl.fast_lds, pl.FNT, st);
  }
  if (narrow_mix<J>(p))
    return em ? launch_chunk_dir<Chunk<J, R, FWD, LOGSR, MARG, 2, kInEmit>>(pl, p, pl.fast_lds, pl.FNT, st)
              : launch_chunk_dir<Chunk<J, R, FWD, LOGSR, MARG, 2, kInCum>>(pl, p, pl.fast_lds, pl.FNT, st);
  return em ? launch_chunk_dir<Chunk<J, R, FWD, LOGSR, MARG, 4, kInEmit>>(pl, p, pl.fast_lds, pl.FNT, st)
            : launch_chunk_dir<Chunk<J, R, FWD, LOGSR, MARG, 4, kInCum>>(pl, p, pl.fast_lds, pl.FNT, st);
}

template <int J, int R>
int launch_fast_jr(const Plan& pl, const ScanParams& p, bool fwd, hipStream_t st) {
  return fwd ? launch_chunk_any<J, R, true, true, false>(pl, p, st) : launch_chunk_any<J, R, false, true, false>(pl, p, st);
}

// Backward log scan with the segment marginals fused (16-lane groups).
template <int R>
int launch_fused_r(const Plan& pl, const ScanParams& p, hipStream_t st) {
  return launch_chunk_any<16, R, false, true, true>(pl, p, st);
}

// Max-semiring forward with backpointers (factorised Viterbi).
template <int J, int R>
int launch_fast_max_jr(const Plan& pl, const ScanParams& p, hipStream_t st) {
  return launch_chunk_any<J, R, true, false, false>(pl, p, st);
}

}  // namespace fastscan
}  // namespace tsm
