// C ABI of libtsm_hip.so (declarations and documentation in include/tsm_hip.h).
// Host side only: validation, launch plan, workspace carving, kernel launches.
// Nothing here allocates device memory; all state lives in caller buffers.

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdlib.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>

#include "../../include/tsm_hip.h"
#include "tsm_internal.hpp"

namespace tsm {
size_t viterbi_lds_bytes(int C, int Kmax, int RS, int has_ps);
}

namespace {

using tsm::Plan;

thread_local std::string g_err;

// Default acceptance threshold of speculative chunks (log2 units); see spec_tolerance().
constexpr float kSpecTol = 4.0e-6f;

// Sequences at least this long get the separate marginals' coverage pass (block
// scales); shorter ones drift far below the gradient tolerance.
constexpr int kCoverageMinT = 65536;

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return code;
}

int hip_fail(int e, const char* where) {
  return fail(TSM_ERR_HIP, "%s: HIP error %d (%s)", where, e, hipGetErrorString((hipError_t)e));
}

struct DeviceInfo {
  int n_cu = 256;
  int max_lds = 160 * 1024;
};

DeviceInfo device_info() {
  DeviceInfo d;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) {
    (void)hipGetLastError();
    return d;
  }
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0) d.n_cu = v;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess && v > 0)
    d.max_lds = v;
  (void)hipGetLastError();
  return d;
}

int pow2_lanes(int C) {
  int J = 64;
  while (J > 1 && (int64_t)C * J > 512) J >>= 1;
  return J;
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// (lanes per label, durations per lane) pairs compiled for the fast scan
// (tsm_fast_j*.hip).
bool fast_instantiated(int J, int R) {
  if (R < 1) return false;
  switch (J) {
    case 8:
    case 32: return R <= 16 || R == 20 || R == 24 || R == 28 || R == 32;
    case 16: return R <= 32;
    case 64: return R <= 8;
    default: return false;
  }
}

// Register-resident log-semiring scan: pick the lane-group size J whose padded
// duration range and wave count give the least work per step; leave p.fast = 0
// when no instance fits.  TSM_SCAN_PATH=generic in the environment disables
// the fast path (used by the tests to exercise the generic kernels).
void plan_fast(Plan& p, const DeviceInfo& di, int fj_only = 0) {
  p.fast = 0;
  const char* env = getenv("TSM_SCAN_PATH");
  if (env != nullptr && strcmp(env, "generic") == 0) return;
  double best = 1e300;
  const char* jenv = getenv("TSM_FAST_J");  // diagnostics: only this lane-group size
  const int jonly = fj_only != 0 ? fj_only : (jenv != nullptr ? atoi(jenv) : 0);
  // Fewer warm-up-long pieces of the sequences than CUs: the chunks are few and
  // each step's latency is the time, not the wave count.  16-lane groups then win
  // where they fit (shorter per-lane chains than 8 lanes, and the backward with
  // fused marginals; measured at B=4, T=1000, C=24, K=100: loss + backward 1.13 ->
  // 0.94 ms, decode 1.38 -> 1.34 ms; 32 lanes slower than either).
  const int64_t pieces = (int64_t)p.B * std::max<int64_t>(1, (int64_t)p.T / (p.Kmax + 64));
  const bool latency_bound = pieces < (int64_t)di.n_cu;
  for (int J : {8, 16, 32, 64}) {
    if (jonly != 0 && J != jonly) continue;
    if (p.C > 4 * J) continue;  // the label mix handles at most 4 labels per lane
    int R = (p.Kmax + J - 1) / J;
    while (R <= 32 && !fast_instantiated(J, R)) ++R;
    if (R > 32) continue;
    const int NT = (int)cdiv((int64_t)p.C * J, 64) * 64;
    if (NT > (R > 16 ? 512 : 1024)) continue;  // the kernels' launch bounds
    const int KP = J * R;
    const int RS = p.Kmax + 2;  // levels of the positions a step reads (pos % RS)
    // linear ring of RL > KP entries, compacted every RL - KP steps: about 2*KP+1
    // entries, fewer when LDS is short (at least 32 steps between compactions).
    // RL % 32 == J % 32 puts the label rows of a half-wave on distinct banks.
    auto ring_fits = [&](int rl, int per) { return (size_t)per * tsm::fast_lds_layout(p.C, rl, RS, 0).total <= (size_t)di.max_lds; };
    auto bank_down = [&](int rl) { while (rl > 0 && rl % 32 != J % 32) --rl; return rl; };
    // the longest ring (<= 2*KP+1 entries) of which `per` fit one CU, 0 if none does
    auto ring_for = [&](int per) {
      int rl = bank_down(2 * KP + 1 + 31);
      if (ring_fits(rl, per)) return rl;
      while (rl > KP && !ring_fits(rl, per)) --rl;
      rl = bank_down(rl);
      return rl < KP + 33 ? 0 : rl;
    };
    int RL = ring_for(1);
    if (RL == 0) continue;
    // 16-lane plans: the fused-marginal beta scan's operand stage behind the rings,
    // batches of 16, 8 or 4 steps (the longest that fits), else batches of 4 with
    // the ring shortened (down to the same 32 steps between compactions)
    size_t fstage = 0;
    int fsb = 0;
    if (J == 16) {
      auto stage_bytes = [&](int sb) { return (size_t)(NT / J) * (2 * sb + 1) * 16; };
      for (int sb : {16, 8, 4}) {
        if (tsm::fast_lds_layout(p.C, RL, RS, stage_bytes(sb)).total <= (size_t)di.max_lds) {
          fstage = stage_bytes(sb);
          fsb = sb;
          break;
        }
      }
      if (fsb == 0) {
        int rl = RL;
        while (rl >= KP + 33 && tsm::fast_lds_layout(p.C, rl, RS, stage_bytes(4)).total > (size_t)di.max_lds)
          rl = bank_down(rl - 1);
        if (rl >= KP + 33) {
          RL = rl;
          fstage = stage_bytes(4);
          fsb = 4;
        }
      }
    }
    const size_t lds = tsm::fast_lds_layout(p.C, RL, RS, fstage).total;
    // rings for two chunks per CU (used when the compiled kernel also leaves
    // registers for a second workgroup)
    const int RL2 = ring_for(2);
    double cost = (double)((NT / 64 + 3) / 4) * (R + 12);  // waves per SIMD x work per wave
    if (latency_bound && J == 16 && fsb > 0) cost = 0.0;
    if (cost < best) {
      best = cost;
      p.fast = 1;
      p.FJ = J;
      p.FR = R;
      p.FNT = NT;
      p.FRS = RS;
      p.FRL = RL;
      p.fast_lds = lds;
      p.fstage = fstage;
      p.FSB = fsb;
      p.FRL2 = RL2;
      p.fast_lds2 = RL2 > 0 ? tsm::fast_lds_layout(p.C, RL2, RS, 0).total : 0;
    }
  }
}

// Cooperative log-semiring scan when no single-block plan holds the rings:
// the smallest group size G (fewest blocks exchanging per step) whose per-block
// rings fit LDS, 16 lanes per label, durations per lane rounded up to a
// multiple of 8 (the compiled instances), at most 128 labels.  The group count
// is what stays co-resident with one block per CU.
void plan_coop(Plan& p, const DeviceInfo& di) {
  p.coop = 0;
  const char* env = getenv("TSM_SCAN_PATH");
  if (env != nullptr && strcmp(env, "generic") == 0) return;
  if (p.C > 128) return;
  const int J = 16;
  int R = (p.Kmax + J - 1) / J;
  R = (R + 7) / 8 * 8;
  if (R > 32) return;
  const int KP = J * R;
  const int RS = p.Kmax + 2;  // levels of the positions a step reads (pos % RS)
  auto bank_down = [&](int rl) { while (rl > 0 && rl % 32 != J % 32) --rl; return rl; };
  for (int G : {2, 4, 8, 16}) {
    const int CL = (p.C + G - 1) / G;
    // the instances' launch bounds (tsm_coopscan.hpp), and every member owns a label
    if (CL * J > (R > 16 ? 256 : 512) || CL * (G - 1) >= p.C) continue;
    // linear ring (as the single-block scan's): up to 2*KP+1 entries, at least
    // 32 steps between compactions
    int RL = bank_down(2 * KP + 1 + 31);
    while (RL > KP && tsm::coop_lds_layout(CL, p.C, RL, RS).total > (size_t)di.max_lds) --RL;
    RL = bank_down(RL);
    if (RL < KP + 33) continue;
    const size_t lds = tsm::coop_lds_layout(CL, p.C, RL, RS).total;
    const int NQ = di.n_cu / G;
    if (NQ < 1) continue;
    p.coop = 1;
    p.CG = G;
    p.CCL = CL;
    p.CR = R;
    p.CNT = (int)cdiv((int64_t)CL * J, 64) * 64;
    p.CRS = RS;
    p.CRL = RL;
    p.coop_lds = lds;
    // members share blockIdx % 8 (one XCD) when whole groups of 8 fit the CUs
    p.cxmap = (di.n_cu % (8 * G) == 0) ? 1 : 0;
    p.CNQ = NQ;
    p.CGRID = NQ * G;
    return;
  }
}

// Duration-dependent transitions: dense scans (J lanes per label, transitions
// in LDS when they fit) and the dense marginal kernel (label groups of G lanes,
// blocks of TB >= Kmax start positions whose start / end sums fit in LDS).
int plan_dense(Plan& p, const DeviceInfo& di) {
  const int C = p.C, Kmax = p.Kmax;
  if (C > 128)
    return fail(TSM_ERR_UNSUPPORTED, "duration-dependent transitions support C <= 128 (got C=%d)", C);
  int kp2 = 4;
  while (kp2 < Kmax) kp2 <<= 1;
  int J = 4;
  for (int cand : {64, 16})
    if (C * cand <= 1024 && cand <= kp2) {
      J = cand;
      break;
    }
  p.DJ = J;
  p.DNT = (int)cdiv((int64_t)C * J, 64) * 64;
  p.DRS = Kmax + 1;
  p.dtrl = 1;
  size_t lds = tsm::dense_lds_layout(C, Kmax, p.DRS, 1).total;
  if (lds > (size_t)di.max_lds) {
    p.dtrl = 0;
    lds = tsm::dense_lds_layout(C, Kmax, p.DRS, 0).total;
    if (lds > (size_t)di.max_lds)
      return fail(TSM_ERR_UNSUPPORTED, "duration-dependent transitions: C=%d, K=%d needs %zu bytes of LDS (> %d)", C,
                  p.K, lds, di.max_lds);
  }
  p.dense_lds = lds;
  int G = 1;
  while (G < C && G < 64) G <<= 1;
  p.DG = G;
  p.DNTM = (int)std::min<int64_t>(1024, cdiv((int64_t)C * G, 64) * 64);
  // about two blocks per CU, at most 512 MiB of fp64 transition partials
  const int64_t per_block = (int64_t)Kmax * C * C * 8;
  int64_t NB = cdiv(2 * (int64_t)di.n_cu, p.B);
  NB = std::min<int64_t>(NB, std::max<int64_t>(1, p.T / std::max(Kmax, 64)));
  NB = std::min<int64_t>(NB, std::max<int64_t>(1, ((int64_t)512 << 20) / (per_block * p.B)));
  NB = std::max<int64_t>(NB, 1);
  int64_t TB = cdiv(p.T, NB);
  if (TB < Kmax) TB = Kmax;
  size_t ml = tsm::dense_marg_lds_layout(C, Kmax, (int)TB).total;
  while (ml > (size_t)di.max_lds && TB > Kmax) {
    TB = std::max<int64_t>(Kmax, TB / 2);
    ml = tsm::dense_marg_lds_layout(C, Kmax, (int)TB).total;
  }
  if (ml > (size_t)di.max_lds)
    return fail(TSM_ERR_UNSUPPORTED, "duration-dependent transitions: marginals for C=%d, K=%d need %zu bytes of LDS (> %d)",
                C, p.K, ml, di.max_lds);
  p.DTB = (int)TB;
  p.DNB = (int)cdiv(p.T, TB);
  p.dmarg_lds = ml;
  p.dense = 1;
  return TSM_OK;
}

// Thread mapping, rings, chunking and marginal blocking for a problem shape.
// trows > 0: the transition is (trows, C, C), one matrix per duration index.
// fj_only != 0: register-resident scans with that many lanes per label only
int make_plan(int64_t B, int64_t T, int64_t C, int64_t K, int has_ps, int has_pe, int64_t trows, Plan* out,
              int fj_only = 0) {
  if (B < 1 || T < 1 || C < 1 || K < 1) return fail(TSM_ERR_INVALID, "need B, T, C, K >= 1 (got %lld, %lld, %lld, %lld)",
                                                    (long long)B, (long long)T, (long long)C, (long long)K);
  if (C > 512) return fail(TSM_ERR_UNSUPPORTED, "num_classes C=%lld > 512 is not supported", (long long)C);
  if (K > 65535) return fail(TSM_ERR_UNSUPPORTED, "max_duration K=%lld > 65535 is not supported", (long long)K);
  if (T > (int64_t)1 << 30) return fail(TSM_ERR_UNSUPPORTED, "T=%lld is too long", (long long)T);
  if (trows < 0) return fail(TSM_ERR_INVALID, "trans_rows must be >= 0 (got %lld)", (long long)trows);
  const DeviceInfo di = device_info();
  Plan p{};
  p.B = (int)B;
  p.T = (int)T;
  p.C = (int)C;
  p.K = (int)K;
  p.Kmax = (int)std::max<int64_t>(K - 1, 1);
  p.has_ps = has_ps;
  p.has_pe = has_pe;
  p.J = pow2_lanes(p.C);
  p.NT = (int)cdiv((int64_t)p.C * p.J, 64) * 64;
  // durations per lane and padded duration range
  p.R = (p.Kmax + p.J - 1) / p.J;
  p.KP = p.J * p.R;
  // ring slots: >= Kmax+2 and > KP; RS % 32 == J % 32 spreads label groups over LDS banks
  int rs = std::max(p.Kmax + 2, p.KP + 1);
  while (rs % 32 != p.J % 32) ++rs;
  p.RS = rs;
  // ring row: >= RS + KP, and RL % 64 == J % 64 so the 64/J label groups of a
  // wave start on different LDS banks
  int rl = p.RS + p.KP;
  while (rl % 64 != p.J % 64) ++rl;
  p.RL = rl;
  const int has_proj = (has_ps || has_pe) ? 1 : 0;
  (void)has_proj;
  size_t lds = tsm::scan_lds_layout(p.C, p.KP, p.RS, p.RL, 0).total;
  p.global_rings = 0;
  if (lds > (size_t)di.max_lds) {
    p.global_rings = 1;
    lds = tsm::scan_lds_layout(p.C, p.KP, p.RS, p.RL, 1).total;
    if (lds > (size_t)di.max_lds)
      return fail(TSM_ERR_UNSUPPORTED, "C=%d needs %zu bytes of LDS (> %d)", p.C, lds, di.max_lds);
  }
  // register-resident duration terms when a lane has at most 32 of them
  p.RMAX = (!p.global_rings && p.R <= 32) ? 32 : 0;
  p.scan_lds = lds;
  // chunking: about one work item per CU; chunks long enough that the warm-up
  // (W steps) costs at most ~25%.  When that leaves most CUs idle (few, short
  // sequences), a chunk's step count is the time: chunks down to one warm-up
  // long, about 2W steps each instead of up to T.
  p.W = p.Kmax + 64;
  const int64_t min_lc = std::max<int64_t>(4 * (int64_t)p.W, 128);
  int64_t P = cdiv(di.n_cu, B);
  P = std::min<int64_t>(P, std::max<int64_t>(1, T / min_lc));
  if (B * P * 2 <= di.n_cu) {
    const int64_t short_lc = std::max<int64_t>(p.W, 128);
    P = std::min<int64_t>(cdiv(di.n_cu, B), std::max<int64_t>(1, T / short_lc));
  }
  P = std::max<int64_t>(P, 1);
  p.P = (int)P;
  p.Lc = (int)cdiv(T, P);
  // marginal kernel: label blocks so the rings fit in LDS
  int CB = p.C;
  for (;;) {
    const int JM = pow2_lanes(CB);
    const size_t ml = tsm::marg_lds_layout(p.C, CB, p.Kmax, p.RS, has_pe).total;
    if (ml <= (size_t)di.max_lds) {
      p.CB = CB;
      p.JM = JM;
      p.NTM = (int)cdiv((int64_t)CB * JM, 64) * 64;
      p.marg_lds = ml;
      break;
    }
    if (CB == 1) return fail(TSM_ERR_UNSUPPORTED, "marginal kernel does not fit LDS (K=%d)", p.K);
    CB = (CB + 1) / 2;
  }
  p.NCB = (int)cdiv(p.C, p.CB);
  int64_t NB = cdiv(2 * (int64_t)di.n_cu, B * p.NCB);
  NB = std::min<int64_t>(NB, std::max<int64_t>(1, T / std::max(p.Kmax, 64)));
  NB = std::max<int64_t>(NB, 1);
  int64_t TB = cdiv(T, NB);
  if (TB < p.Kmax) {
    TB = p.Kmax;
    NB = cdiv(T, TB);
  }
  p.NB = (int)NB;
  p.TB = (int)TB;
  p.trows = (int)trows;
  if (trows > 0) {
    if (trows < p.Kmax + 1)
      return fail(TSM_ERR_INVALID,
                  "duration-dependent transitions are indexed by duration 1..%d: need trans_rows >= %d, got %lld",
                  p.Kmax, p.Kmax + 1, (long long)trows);
    const int rc = plan_dense(p, di);
    if (rc) return rc;
    *out = p;
    return TSM_OK;
  }
  plan_fast(p, di, fj_only);
  if (!p.fast) plan_coop(p, di);
  if (p.coop) {
    // fewer, longer chunks (one per group): a 4x longer warm-up up front, which
    // long segment durations need, at a small share of the chunk
    p.W = 4 * (p.Kmax + 64);
    const int64_t min_lc = 4 * (int64_t)p.W;
    int64_t P = cdiv(p.CNQ, B);
    P = std::max<int64_t>(1, std::min<int64_t>(P, std::max<int64_t>(1, T / min_lc)));
    p.P = (int)P;
    p.Lc = (int)cdiv(T, P);
  }
  if (p.fast) {
    // the register-resident scan keeps a chunk's state in LDS: when several fit
    // on a CU, give each CU that many chunks (up to 8: their step chains are
    // latency-bound and overlap on a SIMD), chunks at least 2W long (measured at
    // B=32, T=10^4, C=8, K=1: 32 chunks 0.79 ms, 64 chunks 0.62 ms fwd+bwd)
    const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(8, (int64_t)di.max_lds / (int64_t)p.fast_lds));
    const int64_t min_lc = std::max<int64_t>(2 * (int64_t)p.W, 128);
    int64_t P2 = cdiv((int64_t)di.n_cu * per_cu, B);
    P2 = std::max<int64_t>(1, std::min<int64_t>(P2, std::max<int64_t>(1, T / min_lc)));
    if (P2 > p.P) {
      p.P = (int)P2;
      p.Lc = (int)cdiv(T, P2);
    }
  }
  if (const char* pe = getenv("TSM_PLAN_P")) {
    // diagnostics: force the chunk count of the register-resident scans
    const int64_t want = atoll(pe);
    if (p.fast && want >= 1) {
      p.P = (int)std::max<int64_t>(1, std::min<int64_t>(want, T / ((int64_t)p.Kmax + 1)));
      p.Lc = (int)cdiv(T, p.P);
    }
  }
  p.mfast = 0;
  const char* env = getenv("TSM_SCAN_PATH");
  const bool generic_only = env != nullptr && strcmp(env, "generic") == 0;
  if (!generic_only && p.C <= 128 && (p.Kmax + 15) / 16 <= 32) {
    // register-resident marginals: 16 lanes per label, one wavefront of 4 labels
    // per workgroup, rings hold the KP positions of a step plus the 16 staged ahead;
    // above 64 labels the instances come in steps of 4 durations per lane
    const int J = 16, MR = p.C > 64 ? ((p.Kmax + 15) / 16 + 3) / 4 * 4 : (p.Kmax + 15) / 16, KP = J * MR;
    const int CBm = 64 / J;
    const int RSm = std::max(p.Kmax + 2, KP + J);
    // linear ring of KP + 2 or 3 batches of 16 entries (moved every few batches),
    // RL % 32 == 16 so the four label rows of a wave fall on distinct banks
    int RLm = KP + 2 * J;
    if (RLm % 32 != 16) RLm += J;
    const size_t lds = tsm::margfast_lds_layout(CBm, RLm, J, p.C).total;
    if (lds <= (size_t)di.max_lds) {
      p.mfast = 1;
      p.MR = MR;
      p.MRS = RSm;
      p.MRL = RLm;
      p.CB = CBm;
      p.NCB = (int)cdiv(p.C, CBm);
      p.JM = J;
      p.NTM = 64;
      p.marg_lds = lds;
      // about two rounds of workgroups over the CUs (as many per CU as LDS allows),
      // blocks at least 4*KP positions long (staging overhead <= 25%)
      const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(8, (int64_t)di.max_lds / (int64_t)lds));
      int64_t nbm = cdiv(2 * (int64_t)di.n_cu * per_cu, (int64_t)p.B * p.NCB);
      nbm = std::min<int64_t>(nbm, std::max<int64_t>(1, T / (4 * (int64_t)KP)));
      nbm = std::max<int64_t>(nbm, 1);
      int64_t tbm = cdiv(T, nbm);
      if (tbm < p.Kmax) {
        tbm = p.Kmax;
        nbm = cdiv(T, tbm);
      }
      if (const char* ne = getenv("TSM_MARG_NB")) {
        // diagnostics: force the position blocks of the register-resident marginals
        const int64_t want = atoll(ne);
        if (want >= 1) {
          tbm = std::max<int64_t>(p.Kmax, cdiv(T, want));
          nbm = cdiv(T, tbm);
        }
      }
      p.NB = (int)nbm;
      p.TB = (int)tbm;
    }
  }
  // marginals fused into the backward scan: the register-resident scan with
  // 16-lane groups (TSM_MARGINAL_PATH=separate keeps the separate kernel).  (The
  // same fusion in the cooperative scan was measured slower at cfg5: one wave
  // per SIMD there, so the extra per-term work lands on the step's critical path.)
  p.mfused = 0;
  const char* menv = getenv("TSM_MARGINAL_PATH");
  const bool separate = menv != nullptr && strcmp(menv, "separate") == 0;
  if (!separate && p.fast && p.FJ == 16 && p.FSB > 0) {
    p.mfused = 1;
    // transition gradient: about eight blocks per CU, at least 64 starts (one staged
    // batch of rows) each; short sequences get more, shorter blocks (B=4, T=1000:
    // 16 blocks per sequence, 44 -> 12 us)
    int64_t gnb = cdiv(8 * (int64_t)di.n_cu, (int64_t)p.B);
    gnb = std::max<int64_t>(1, std::min<int64_t>(gnb, cdiv(T, 64)));
    p.GTB = (int)cdiv(T, gnb);
    p.GNB = (int)cdiv(T, p.GTB);
  }
  // Two chunks per CU with the smaller rings, for each fast scan direction whose
  // kernel allows it.  A second workgroup is placed on a CU only when every SIMD
  // has registers for the waves the workgroup puts on it (a six-wave workgroup
  // puts two on a SIMD, so at most 128 VGPRs); otherwise the two would run one
  // after the other, with twice the warm-up.  TSM_SCAN_CHUNKS=single turns this
  // off; =dual (tests) takes up to twice the chunks of the plan, each at least
  // Kmax+1 positions long, so that small problems exercise the same path.
  p.regsF = p.regsB = p.regsV = -1;
  const char* cenv = getenv("TSM_SCAN_CHUNKS");
  const bool single = cenv != nullptr && strcmp(cenv, "single") == 0;
  const bool force = cenv != nullptr && strcmp(cenv, "dual") == 0;
  if (p.fast && p.FRL2 > 0 && !single) {
    const int64_t min_lc = std::max<int64_t>(4 * (int64_t)p.W, 128);
    int64_t P2 = cdiv(2 * (int64_t)di.n_cu, B);
    P2 = std::max<int64_t>(1, std::min<int64_t>(P2, std::max<int64_t>(1, T / min_lc)));
    if (force) P2 = std::min<int64_t>(2 * (int64_t)p.P, std::max<int64_t>(1, T / ((int64_t)p.Kmax + 1)));
    if (P2 > p.P) {
      Plan q = p;
      q.FRL = p.FRL2;
      q.fast_lds = p.fast_lds2;
      auto pair_fits = [&](int regs) {
        if (regs <= 0) return 0;
        const int alloc = (regs + 7) / 8 * 8;
        const int per_simd = (p.FNT / 64 + 3) / 4;
        return 2 * per_simd * alloc <= 512 ? 1 : 0;
      };
      p.regsF = tsm::fast_scan_regs(q, 0);
      p.regsB = tsm::fast_scan_regs(q, 1);
      p.regsV = tsm::fast_scan_regs(q, 2);
      p.dualF = pair_fits(p.regsF);
      p.dualB = p.mfused ? 0 : pair_fits(p.regsB);
      p.dualV = pair_fits(p.regsV);
      if (p.dualF || p.dualB || p.dualV) {
        p.P2 = (int)P2;
        p.Lc2 = (int)cdiv(T, P2);
      }
    }
  }
  if (p.P2 == 0) p.dualF = p.dualB = p.dualV = 0;
  *out = p;
  return TSM_OK;
}

// The plan of a fast scan direction that runs two chunks per CU.
Plan dual_plan(const Plan& pl) {
  Plan q = pl;
  q.P = pl.P2;
  q.Lc = pl.Lc2;
  q.FRL = pl.FRL2;
  q.fast_lds = pl.fast_lds2;
  return q;
}

// Bump allocator over the caller's workspace (256-byte aligned pieces).
struct Carver {
  char* base;
  size_t off = 0;
  explicit Carver(void* b) : base(static_cast<char*>(b)) {}
  template <typename T>
  T* take(size_t n) {
    off = (off + 255) & ~size_t(255);
    T* p = base ? reinterpret_cast<T*>(base + off) : nullptr;
    off += n * sizeof(T);
    return p;
  }
};

struct ScanWs {
  float *st_spec, *st_end, *fin, *gring;
  double *lv_spec, *lv_end, *offs, *vstat, *fin_lvl, *z2;
  int* status;
  int* vflag;
  unsigned long long* xch;
  int* xabort;
};

// (Sized for the larger of the plan's two chunkings, so that either fits.)
// generic_rings: the generic scan kernels may run (the max semiring, or a log
// plan without the register-resident or cooperative scans); only they keep
// rings in the workspace when LDS is too small.
ScanWs carve_scan(Carver& cv, const Plan& p, bool generic_rings = true) {
  ScanWs w;
  const size_t items = (size_t)p.B * std::max(p.P, p.P2);
  w.st_spec = cv.take<float>(items * p.Kmax * p.C);
  w.st_end = cv.take<float>(items * p.Kmax * p.C);
  w.lv_spec = cv.take<double>(items * p.Kmax);
  w.lv_end = cv.take<double>(items * p.Kmax);
  w.offs = cv.take<double>(items);
  w.vstat = cv.take<double>(2 * items);
  w.status = cv.take<int>(items);
  w.vflag = cv.take<int>(1);
  w.fin = cv.take<float>((size_t)p.B * p.C);
  w.fin_lvl = cv.take<double>(p.B);
  w.z2 = cv.take<double>(p.B);
  w.gring = (p.global_rings && generic_rings && !p.dense)
                ? cv.take<float>(items * tsm::scan_gring_floats(p.C, p.KP, p.RL))
                : nullptr;
  w.xch = p.coop ? cv.take<unsigned long long>((size_t)p.CNQ * 2 * p.C) : nullptr;
  w.xabort = p.coop ? cv.take<int>(1) : nullptr;
  return w;
}

// Acceptance threshold of a speculative chunk: the spread (max - min, log2
// units) of exact minus speculative boundary state.  TSM_SPEC_TOL overrides it
// (diagnostics and tests).
float spec_tolerance() {
  const char* e = getenv("TSM_SPEC_TOL");
  if (e != nullptr && *e != '\0') {
    const float v = (float)atof(e);
    if (v > 0.0f) return v;
  }
  return kSpecTol;
}

tsm::ScanParams scan_params(const Plan& pl, const ScanWs& w, const float* cum, const float* tr, const float* db,
                            const int64_t* len, const float* ps, const float* pe) {
  tsm::ScanParams p{};
  p.cum = cum;
  p.trans = tr;
  p.db = db;
  p.lengths = len;
  p.ps = ps;
  p.pe = pe;
  p.B = pl.B;
  p.T = pl.T;
  p.C = pl.C;
  p.K = pl.K;
  p.Kmax = pl.Kmax;
  p.RS = pl.RS;
  p.R = pl.R;
  p.KP = pl.KP;
  p.RL = pl.RL;
  p.P = pl.P;
  p.Lc = pl.Lc;
  p.W = pl.W;
  p.tol = spec_tolerance();
  p.st_spec = w.st_spec;
  p.st_end = w.st_end;
  p.lv_spec = w.lv_spec;
  p.lv_end = w.lv_end;
  p.offs = w.offs;
  p.vstat = w.vstat;
  p.status = w.status;
  p.vflag = w.vflag;
  p.fin = w.fin;
  p.fin_lvl = w.fin_lvl;
  p.z2 = w.z2;
  p.gring = w.gring;
  p.xch = w.xch;
  p.xabort = w.xabort;
  p.G = pl.CG;
  p.CL = pl.CCL;
  p.NQ = pl.CNQ;
  p.xmap = pl.cxmap;
  return p;
}

int check_common(const float* cum, const float* tr, const float* db, const int64_t* len, int semiring) {
  if (!cum || !tr || !db || !len) return fail(TSM_ERR_INVALID, "cum_scores, transition, duration_bias and lengths are required");
  if (semiring != TSM_SEMIRING_LOG && semiring != TSM_SEMIRING_MAX)
    return fail(TSM_ERR_INVALID, "semiring must be TSM_SEMIRING_LOG (0) or TSM_SEMIRING_MAX (1), got %d", semiring);
  return TSM_OK;
}

// log2-scaled transition tables of both directions (duration-dependent transitions)
struct DenseTr {
  float *trf, *trb;
};

DenseTr carve_dense(Carver& cv, const Plan& p) {
  DenseTr d{nullptr, nullptr};
  if (!p.dense) return d;
  d.trf = cv.take<float>((size_t)p.Kmax * p.C * p.C);
  d.trb = cv.take<float>((size_t)p.Kmax * p.C * p.C);
  return d;
}

// Marginal blocking of the plan's marginal kernel
int marg_nb(const Plan& p) { return p.dense ? p.DNB : p.NB; }
int marg_tb(const Plan& p) { return p.dense ? p.DTB : p.TB; }
size_t tr_part_len(const Plan& p) {
  return (size_t)p.B * marg_nb(p) * (p.dense ? (size_t)p.Kmax : 1) * p.C * p.C;
}

// The forward runs a generic scan kernel unless a register-resident plan covers
// its semiring (log only) or the plan is cooperative (both semirings).
bool forward_generic(const Plan& pl, int semiring) {
  return !pl.coop && (semiring != TSM_SEMIRING_LOG || !pl.fast);
}

size_t forward_ws_bytes(const Plan& pl, int semiring) {
  Carver cv(nullptr);
  carve_scan(cv, pl, forward_generic(pl, semiring));
  carve_dense(cv, pl);
  return cv.off + 256;
}

// Backward workspace.  Separate marginals: the beta table, the scan workspace,
// end / start sums and the marginal kernel's block partials.  Fused marginals
// (mfused): u, the scan workspace, end / start sums, and per backward chunk the
// halo rows, duration sums and frame estimate; transition partials per row block.
struct BwdWs {
  float *bval = nullptr, *uval = nullptr, *e_own, *s_out, *halo;
  double *blvl = nullptr, *db_part, *tr_part, *mframe = nullptr, *bscale = nullptr;
  ScanWs scan;
  DenseTr dt;
};

BwdWs carve_backward(Carver& cv, const Plan& pl) {
  BwdWs w;
  const size_t rows = (size_t)pl.B * (pl.T + 1);
  if (pl.mfused) {
    const size_t items = (size_t)pl.B * pl.P;
    w.uval = cv.take<float>(rows * pl.C);
    w.scan = carve_scan(cv, pl);
    w.e_own = cv.take<float>(rows * pl.C);
    w.s_out = cv.take<float>(rows * pl.C);
    w.halo = cv.take<float>(items * pl.Kmax * pl.C);
    w.db_part = cv.take<double>(items * pl.Kmax * pl.C);
    w.mframe = cv.take<double>(items);
    w.tr_part = cv.take<double>((size_t)pl.B * pl.GNB * pl.C * pl.C);
  } else {
    w.bval = cv.take<float>(rows * pl.C);
    w.blvl = cv.take<double>(rows);
    w.scan = carve_scan(cv, pl);
    w.e_own = cv.take<float>(rows * pl.C);
    w.s_out = cv.take<float>(rows * pl.C);
    w.halo = cv.take<float>((size_t)pl.B * marg_nb(pl) * pl.Kmax * pl.C);
    w.db_part = cv.take<double>((size_t)pl.B * marg_nb(pl) * pl.Kmax * pl.C);
    w.tr_part = cv.take<double>(tr_part_len(pl));
    w.bscale = cv.take<double>((size_t)pl.B * marg_nb(pl));
  }
  w.dt = carve_dense(cv, pl);
  return w;
}

// (with fused marginals, also enough for the separate layout that a
// max-semiring backward uses)
size_t backward_ws_bytes(const Plan& pl) {
  Carver cv(nullptr);
  carve_backward(cv, pl);
  size_t n = cv.off;
  if (pl.mfused) {
    Plan q = pl;
    q.mfused = 0;
    Carver cs(nullptr);
    carve_backward(cs, q);
    n = std::max(n, cs.off);
  }
  return n + 256;
}

// Viterbi workspace: backpointers, final labels, and the scan workspace of the
// factorised algorithm (sized for whichever algorithm a call selects).
size_t viterbi_ws_bytes(const Plan& pl, int with_tb) {
  Carver cv(nullptr);
  if (with_tb) cv.take<int32_t>((size_t)pl.B * (pl.T + 1) * pl.C);
  cv.take<int32_t>(pl.B);
  if (pl.fast || pl.coop) {
    carve_scan(cv, pl, false);
    if (with_tb) cv.take<int32_t>((size_t)pl.B * (pl.T + 1) * pl.C);  // factorised backpointers, exact format
  }
  if (with_tb) cv.take<char>(tsm::backtrace_ws_bytes(tsm::backtrace_plan(pl.B, pl.T, pl.C, pl.Kmax), pl.B));
  return cv.off + 256;
}

// Factorised Viterbi is used for algorithm 2, and for algorithm 0 when the
// register-resident or the cooperative scan fits and either the problem has at
// least 2^28 cells (B*T*K*C^2) or the plan cuts each sequence into several
// chunks: the exact kernel runs one workgroup per sequence through all T steps,
// so few long sequences leave most CUs idle (cfg1, B=4 x 1000 steps: 3.2 ms)
// while the chunked scan spreads them over the chip.
bool viterbi_factorised(const Plan& pl, int algorithm) {
  if (algorithm == TSM_VITERBI_EXACT || (!pl.fast && !pl.coop) || pl.dense) return false;
  if (algorithm == TSM_VITERBI_FACTORISED) return true;
  const double cells = (double)pl.B * pl.T * pl.K * (double)pl.C * pl.C;
  return cells >= (double)(1 << 28) || pl.P >= 2;
}

// Gold-path scoring: sizes, LDS of the label window, workspace.
int check_gold(int64_t B, int64_t T, int64_t C, int64_t K, int64_t Kdb) {
  if (B < 1 || T < 1 || C < 1 || K < 1)
    return fail(TSM_ERR_INVALID, "need B, T, C, K >= 1 (got %lld, %lld, %lld, %lld)", (long long)B, (long long)T,
                (long long)C, (long long)K);
  if (Kdb < K || Kdb < 1)
    return fail(TSM_ERR_INVALID, "duration_bias has %lld rows; durations up to K-1 = %lld need >= %lld",
                (long long)Kdb, (long long)(K - 1), (long long)K);
  if (T > (int64_t)1 << 30 || C > 4096 || Kdb * C + C * C > (int64_t)1 << 30)
    return fail(TSM_ERR_UNSUPPORTED, "gold score: sizes too large (T=%lld, C=%lld, K=%lld)", (long long)T,
                (long long)C, (long long)Kdb);
  const DeviceInfo di = device_info();
  if (tsm::gold_lds_bytes((int)K) > (size_t)di.max_lds)
    return fail(TSM_ERR_UNSUPPORTED, "gold score: K=%lld needs a label window larger than LDS", (long long)K);
  return TSM_OK;
}

struct GoldWs {
  double* part;
  int* bad;
  int* cnt;
};

GoldWs carve_gold(Carver& cv, int64_t B, int64_t T, int64_t C, int64_t Kdb) {
  const size_t nch = (size_t)tsm::gold_chunks((int)T);
  GoldWs w;
  w.part = cv.take<double>((size_t)B * nch);
  w.bad = cv.take<int>((size_t)B * nch);
  w.cnt = cv.take<int>((size_t)B * (size_t)(Kdb * C + C * C));
  return w;
}

tsm::GoldParams gold_params(const GoldWs& w, const float* cum, const float* tr, const float* db,
                            const int64_t* labels, const int64_t* len, int64_t B, int64_t T, int64_t C, int64_t K,
                            int64_t Kdb) {
  tsm::GoldParams g{};
  g.cum = cum;
  g.tr = tr;
  g.db = db;
  g.labels = labels;
  g.lengths = len;
  g.B = (int)B;
  g.T = (int)T;
  g.C = (int)C;
  g.K = (int)K;
  g.Kdb = (int)Kdb;
  g.NCH = tsm::gold_chunks((int)T);
  g.part = w.part;
  g.bad = w.bad;
  g.cnt = w.cnt;
  g.NHIST = (int)(Kdb * C + C * C);
  return g;
}

}  // namespace

extern "C" {

int tsm_version(void) { return 100; }

const char* tsm_last_error(void) { return g_err.c_str(); }

int tsm_plan_info(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int has_ps, int has_pe,
                  int64_t* out, int n) {
  Plan p;
  int rc = make_plan(B, T, C, K, has_ps, has_pe, trans_rows, &p);
  if (rc) return rc;
  if (!out) return fail(TSM_ERR_INVALID, "out is NULL");
  const DeviceInfo di = device_info();
  const int64_t vals[] = {p.J, p.NT, p.RS, p.P, p.Lc, p.W, p.global_rings, (int64_t)p.scan_lds, p.NB, p.TB,
                          p.CB, p.NCB, p.JM, p.NTM, (int64_t)p.marg_lds, p.Kmax, di.n_cu, p.R, p.KP, p.RMAX,
                          p.fast, p.FJ, p.FR, p.FNT, (int64_t)p.fast_lds, p.mfast, p.MR,
                          p.dense, p.DJ, p.DNT, p.dtrl, (int64_t)p.dense_lds, p.DG, p.DNTM, p.DNB, p.DTB,
                          (int64_t)p.dmarg_lds, p.coop, p.CG, p.CCL, p.CR, p.CNQ, (int64_t)p.coop_lds,
                          p.mfused, p.GNB, p.GTB, p.P2, p.Lc2, p.FRL2, (int64_t)p.fast_lds2, p.dualF, p.dualB,
                          p.dualV, p.regsF, p.regsB, p.regsV};
  const int m = (int)(sizeof(vals) / sizeof(vals[0]));
  for (int i = 0; i < n && i < m; ++i) out[i] = vals[i];
  return TSM_OK;
}

int tsm_forward_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int semiring, int has_ps,
                          int has_pe, size_t* bytes) {
  if (!bytes) return fail(TSM_ERR_INVALID, "bytes is NULL");
  if (semiring != TSM_SEMIRING_LOG && semiring != TSM_SEMIRING_MAX) return fail(TSM_ERR_INVALID, "bad semiring %d", semiring);
  Plan p;
  int rc = make_plan(B, T, C, K, has_ps, has_pe, trans_rows, &p);
  if (rc) return rc;
  *bytes = forward_ws_bytes(p, semiring);
  return TSM_OK;
}

}  // extern "C"

namespace {

// tsm_forward's work on a given workspace (the caller's, or the static scratch of
// tsm_forward_noalloc).
int forward_impl(const float* cum, const float* tr, const float* db, const int64_t* len, const float* ps,
                 const float* pe, int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int semiring,
                 float* partition, double* log2_partition, float* alpha_hat, double* alpha_level,
                 int32_t* recomputed, void* workspace, size_t ws_bytes, void* stream, const char* what,
                 const float* emit = nullptr) {
  int rc = check_common(emit != nullptr ? emit : cum, tr, db, len, semiring);
  if (rc) return rc;
  if (!partition) return fail(TSM_ERR_INVALID, "partition output is required");
  if ((alpha_hat == nullptr) != (alpha_level == nullptr))
    return fail(TSM_ERR_INVALID, "alpha_hat and alpha_level must both be given or both be NULL");
  Plan pl;
  rc = make_plan(B, T, C, K, ps != nullptr, pe != nullptr, trans_rows, &pl);
  if (rc) return rc;
  const size_t need = forward_ws_bytes(pl, semiring);
  if (!workspace || ws_bytes < need)
    return fail(TSM_ERR_WORKSPACE, "%s: workspace too small: %zu < %zu bytes", what, ws_bytes, need);
  if (semiring == TSM_SEMIRING_LOG && pl.dualF) pl = dual_plan(pl);
  Carver cv(workspace);
  ScanWs w = carve_scan(cv, pl, forward_generic(pl, semiring));
  const DenseTr dt = carve_dense(cv, pl);
  tsm::ScanParams p = scan_params(pl, w, cum, tr, db, len, ps, pe);
  p.emit = emit;
  if (pl.dense) {
    const int e = tsm::launch_dense_prep(pl, tr, dt.trf, dt.trb, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "tsm_forward (transition tables)");
    p.trows = pl.trows;
    p.trx = dt.trf;
  }
  p.val = alpha_hat;
  p.lvl = alpha_level;
  if (log2_partition) p.z2 = log2_partition;
  p.zout = partition;
  p.recomputed = recomputed;
  const int e = tsm::launch_scan_forward(pl, p, semiring, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, what);
  return TSM_OK;
}

// Scratch of tsm_forward_noalloc: a file-scope device array, so a call needs no
// allocation.  Every device holds its own copy (allocated with the code object,
// kept until the process ends).  In host code `scratch` names a host-side
// stand-in, not device memory: its device address on the current device comes
// from hipGetSymbolAddress, once per device, and only that address is used.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxDevices];

}  // namespace

static __device__ __align__(256) unsigned char scratch[TSM_NOALLOC_SCRATCH_BYTES];

namespace {

// The device address of `scratch` on the current device (looked up on the first
// call on each device, with that device current).
int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "tsm_forward_noalloc (hipGetDevice)");
  if (dev < 0 || dev >= kMaxDevices)
    return fail(TSM_ERR_UNSUPPORTED, "tsm_forward_noalloc: device index %d outside [0, %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_dev[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "tsm_forward_noalloc (hipGetSymbolAddress of the scratch array)");
    if (p == nullptr) return fail(TSM_ERR_HIP, "tsm_forward_noalloc: hipGetSymbolAddress returned NULL");
    g_scratch_dev[dev] = p;
  }
  *out = g_scratch_dev[dev];
  return TSM_OK;
}

}  // namespace

extern "C" {

int tsm_forward(const float* cum, const float* tr, const float* db, const int64_t* len, const float* ps,
                const float* pe, int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int semiring,
                float* partition, double* log2_partition, float* alpha_hat, double* alpha_level, int32_t* recomputed,
                void* workspace, size_t ws_bytes, void* stream) {
  return forward_impl(cum, tr, db, len, ps, pe, B, T, C, K, trans_rows, semiring, partition, log2_partition,
                      alpha_hat, alpha_level, recomputed, workspace, ws_bytes, stream, "tsm_forward");
}

int tsm_forward_noalloc(const float* cum, const float* tr, const float* db, const int64_t* len, const float* ps,
                        const float* pe, int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows,
                        int semiring, float* partition, double* log2_partition, float* alpha_hat,
                        double* alpha_level, int32_t* recomputed, void* stream) {
  // plan and size first (host only), so an oversized problem is refused before
  // the scratch is touched
  int rc = check_common(cum, tr, db, len, semiring);
  if (rc) return rc;
  Plan pl;
  rc = make_plan(B, T, C, K, ps != nullptr, pe != nullptr, trans_rows, &pl);
  if (rc) return rc;
  const size_t need = forward_ws_bytes(pl, semiring);
  if (need > (size_t)TSM_NOALLOC_SCRATCH_BYTES)
    return fail(TSM_ERR_UNSUPPORTED,
                "tsm_forward_noalloc: this problem needs %zu bytes of scratch, more than the %zu-byte static "
                "scratch; call tsm_forward with a workspace of tsm_forward_workspace() bytes instead",
                need, (size_t)TSM_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  rc = scratch_address(&ws);
  if (rc) return rc;
  return forward_impl(cum, tr, db, len, ps, pe, B, T, C, K, trans_rows, semiring, partition, log2_partition,
                      alpha_hat, alpha_level, recomputed, ws, (size_t)TSM_NOALLOC_SCRATCH_BYTES, stream,
                      "tsm_forward_noalloc");
}

int tsm_backward_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int has_ps, int has_pe,
                           size_t* bytes) {
  if (!bytes) return fail(TSM_ERR_INVALID, "bytes is NULL");
  Plan p;
  int rc = make_plan(B, T, C, K, has_ps, has_pe, trans_rows, &p);
  if (rc) return rc;
  *bytes = backward_ws_bytes(p);
  return TSM_OK;
}

}  // extern "C"

namespace {

// tsm_backward's work.  emit != null (the emission entry point, on a plan whose
// kernels read projected scores): the kernels take emit in place of cum, and
// grad_cum is the (B, T, C) output with row t >= 1 of the cum gradient at row
// t-1, which the caller turns into the score gradient in place.
int backward_impl(const float* cum, const float* emit, const float* tr, const float* db, const int64_t* len,
                  const float* ps, const float* pe, int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows,
                  int semiring, const float* alpha_hat, const double* alpha_level, const double* log2_partition,
                  const float* grad_output, float* grad_cum, float* grad_tr, float* grad_db, float* grad_ps,
                  float* grad_pe, int32_t* recomputed, void* workspace, size_t ws_bytes, void* stream) {
  int rc = check_common(emit != nullptr ? emit : cum, tr, db, len, semiring);
  if (rc) return rc;
  if (!alpha_hat || !alpha_level || !log2_partition || !grad_output || !grad_cum || !grad_tr || !grad_db)
    return fail(TSM_ERR_INVALID, "alpha_hat, alpha_level, log2_partition, grad_output and the gradient outputs are required");
  if ((ps != nullptr) != (grad_ps != nullptr) || (pe != nullptr) != (grad_pe != nullptr))
    return fail(TSM_ERR_INVALID, "a projection gradient buffer is needed exactly when the projection is given");
  Plan pl;
  rc = make_plan(B, T, C, K, ps != nullptr, pe != nullptr, trans_rows, &pl);
  if (rc) return rc;
  const size_t need = backward_ws_bytes(pl);
  if (!workspace || ws_bytes < need)
    return fail(TSM_ERR_WORKSPACE, "backward workspace too small: %zu < %zu bytes", ws_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  if (semiring != TSM_SEMIRING_LOG) pl.mfused = 0;  // max semiring: the separate marginals
  if (semiring == TSM_SEMIRING_LOG && !pl.mfused && pl.dualB) pl = dual_plan(pl);
  Carver cv(workspace);
  const BwdWs bw = carve_backward(cv, pl);
  const ScanWs& w = bw.scan;
  const DenseTr& dt = bw.dt;
  float* bval = bw.bval;
  double* blvl = bw.blvl;
  float* e_own = bw.e_own;
  float* s_out = bw.s_out;
  float* halo = bw.halo;
  double* db_part = bw.db_part;
  double* tr_part = bw.tr_part;

  tsm::ScanParams p = scan_params(pl, w, cum, tr, db, len, ps, pe);
  p.emit = emit;
  const int shift = emit != nullptr ? 1 : 0;
  if (pl.mfused) {
    tsm::FusedParams f{};
    f.emit = emit;
    f.shift = shift;
    f.lengths = len;
    f.trans = tr;
    f.aval = alpha_hat;
    f.uval = bw.uval;
    f.B = pl.B;
    f.T = pl.T;
    f.C = pl.C;
    f.K = pl.K;
    f.Kmax = pl.Kmax;
    f.P = pl.P;
    f.Lc = pl.Lc;
    f.GNB = pl.GNB;
    f.GTB = pl.GTB;
    f.offs = w.offs;
    f.mframe = bw.mframe;
    f.cum = cum;
    f.db = db;
    f.ps = ps;
    f.alvl = alpha_level;
    f.z2 = log2_partition;
    f.st_end = w.st_end;
    f.lv_end = w.lv_end;
    f.e_own = e_own;
    f.s_out = s_out;
    // the cumulative-score scan takes each end sum from the tables at its owner
    // chunk and writes no halo rows; the emission scan slides them (halo rows)
    f.halo = emit != nullptr ? halo : nullptr;
    f.db_part = db_part;
    f.tr_part = tr_part;
    f.grad_output = grad_output;
    f.grad_cum = grad_cum;
    f.grad_ps = grad_ps;
    f.grad_pe = grad_pe;
    f.grad_tr = grad_tr;
    f.grad_db = grad_db;
    int e = tsm::launch_u_rows(pl, f, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_backward (u rows)");
    p.val = nullptr;
    p.lvl = nullptr;
    p.zout = nullptr;
    p.recomputed = recomputed;
    p.uval = bw.uval;
    p.aval = alpha_hat;
    p.alvl = alpha_level;
    p.mz2 = log2_partition;
    p.e_own = e_own;
    p.s_out = s_out;
    p.halo = halo;
    p.db_part = db_part;
    p.mframe = bw.mframe;
    e = tsm::launch_scan_backward_fused(pl, p, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_backward (beta scan with marginals)");
    e = tsm::launch_fused_finalize(pl, f, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_backward (finalize)");
    return TSM_OK;
  }
  if (pl.dense) {
    const int e = tsm::launch_dense_prep(pl, tr, dt.trf, dt.trb, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_backward (transition tables)");
    p.trows = pl.trows;
    p.trx = dt.trb;
  }
  p.val = bval;
  p.lvl = blvl;
  p.zout = nullptr;
  p.recomputed = recomputed;
  int e = tsm::launch_scan_backward(pl, p, semiring, st);
  if (e != hipSuccess) return hip_fail(e, "tsm_backward (beta scan)");

  tsm::MargParams q{};
  q.cum = cum;
  q.emit = emit;
  q.trans = tr;
  q.db = db;
  q.lengths = len;
  q.ps = ps;
  q.pe = pe;
  q.B = pl.B;
  q.T = pl.T;
  q.C = pl.C;
  q.K = pl.K;
  q.Kmax = pl.Kmax;
  q.RS = pl.mfast ? pl.MRS : pl.RS;
  q.RL = pl.MRL;
  q.NB = marg_nb(pl);
  q.TB = marg_tb(pl);
  q.trows = pl.trows;
  q.trx = dt.trf;
  q.CB = pl.CB;
  q.NCB = pl.NCB;
  q.aval = alpha_hat;
  q.alvl = alpha_level;
  q.bval = bval;
  q.blvl = blvl;
  q.z2 = log2_partition;
  q.e_own = e_own;
  q.s_out = s_out;
  q.halo = halo;
  q.db_part = db_part;
  q.tr_part = tr_part;
  e = tsm::launch_marginals(pl, q, st);
  if (e != hipSuccess) return hip_fail(e, "tsm_backward (marginals)");
  // coverage pass (block scales): long sequences, where the level chains' rounding
  // drift reaches the gradient tolerance; log semiring, static transitions
  const char* cenv = getenv("TSM_COVERAGE");  // diagnostics: =0 skips it
  const bool coverage = semiring == TSM_SEMIRING_LOG && !pl.dense && pl.T >= kCoverageMinT &&
                        (cenv == nullptr || strcmp(cenv, "0") != 0);
  if (coverage) {
    e = tsm::launch_block_coverage(pl, q, bw.bscale, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_backward (coverage)");
  }

  tsm::FinalParams f{};
  f.lengths = len;
  f.B = pl.B;
  f.T = pl.T;
  f.C = pl.C;
  f.K = pl.K;
  f.Kmax = pl.Kmax;
  f.NB = marg_nb(pl);
  f.TB = marg_tb(pl);
  f.trows = pl.trows;
  f.e_own = e_own;
  f.s_out = s_out;
  f.halo = halo;
  f.db_part = db_part;
  f.tr_part = tr_part;
  f.grad_output = grad_output;
  f.grad_cum = grad_cum;
  f.grad_ps = grad_ps;
  f.grad_pe = grad_pe;
  f.grad_tr = grad_tr;
  f.grad_db = grad_db;
  f.bscale = coverage ? bw.bscale : nullptr;
  f.shift = shift;
  e = tsm::launch_finalize(pl, f, st);
  if (e != hipSuccess) return hip_fail(e, "tsm_backward (finalize)");
  return TSM_OK;
}

}  // namespace

extern "C" {

int tsm_backward(const float* cum, const float* tr, const float* db, const int64_t* len, const float* ps,
                 const float* pe, int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int semiring,
                 const float* alpha_hat,
                 const double* alpha_level, const double* log2_partition, const float* grad_output,
                 float* grad_cum, float* grad_tr, float* grad_db, float* grad_ps, float* grad_pe,
                 int32_t* recomputed, void* workspace, size_t ws_bytes, void* stream) {
  if (!cum) return fail(TSM_ERR_INVALID, "cum_scores, transition, duration_bias and lengths are required");
  return backward_impl(cum, nullptr, tr, db, len, ps, pe, B, T, C, K, trans_rows, semiring, alpha_hat, alpha_level,
                       log2_partition, grad_output, grad_cum, grad_tr, grad_db, grad_ps, grad_pe, recomputed,
                       workspace, ws_bytes, stream);
}

int tsm_viterbi_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int with_tb,
                          size_t* bytes) {
  if (!bytes) return fail(TSM_ERR_INVALID, "bytes is NULL");
  Plan p;
  int rc = make_plan(B, T, C, K, 0, 0, trans_rows, &p);
  if (rc) return rc;
  *bytes = viterbi_ws_bytes(p, with_tb);
  return TSM_OK;
}

}  // extern "C"

namespace {

// tsm_viterbi's work.  emit != null (the emission entry point): the factorised
// scan reads the projected scores; the exact kernel is never given them (the
// caller builds cum first for a call that runs it).
int viterbi_impl(const float* cum, const float* emit, const float* tr, const float* db, const int64_t* len,
                 const float* ps, const float* pe, int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows,
                 float* score, int with_tb, int algorithm, int32_t* seg_count, int32_t* segments, void* workspace,
                 size_t ws_bytes, void* stream) {
  int rc = check_common(emit != nullptr ? emit : cum, tr, db, len, TSM_SEMIRING_MAX);
  if (rc) return rc;
  if (!score) return fail(TSM_ERR_INVALID, "score output is required");
  if (with_tb && (!seg_count || !segments)) return fail(TSM_ERR_INVALID, "traceback needs seg_count and segments");
  if (algorithm < TSM_VITERBI_AUTO || algorithm > TSM_VITERBI_FACTORISED)
    return fail(TSM_ERR_INVALID, "algorithm must be TSM_VITERBI_AUTO (0), _EXACT (1) or _FACTORISED (2), got %d",
                algorithm);
  Plan pl;
  rc = make_plan(B, T, C, K, ps != nullptr, pe != nullptr, trans_rows, &pl);
  if (rc) return rc;
  if (algorithm == TSM_VITERBI_FACTORISED && pl.dense)
    return fail(TSM_ERR_UNSUPPORTED, "the factorised Viterbi needs static (C, C) transitions");
  if (algorithm == TSM_VITERBI_FACTORISED && !pl.fast && !pl.coop)
    return fail(TSM_ERR_UNSUPPORTED,
                "the factorised Viterbi needs the register-resident or the cooperative scan (C <= 128, K <= 513)");
  if (viterbi_factorised(pl, algorithm)) {
    const size_t need = viterbi_ws_bytes(pl, with_tb);
    if (!workspace || ws_bytes < need)
      return fail(TSM_ERR_WORKSPACE, "viterbi workspace too small: %zu < %zu bytes", ws_bytes, need);
    if (pl.dualV) pl = dual_plan(pl);
    Carver cv(workspace);
    int32_t* bp = with_tb ? cv.take<int32_t>((size_t)pl.B * (pl.T + 1) * pl.C) : nullptr;
    cv.take<int32_t>(pl.B);
    ScanWs w = carve_scan(cv, pl, false);
    int32_t* bp_exact = with_tb ? cv.take<int32_t>((size_t)pl.B * (pl.T + 1) * pl.C) : nullptr;
    const tsm::BtPlan btp = tsm::backtrace_plan(pl.B, pl.T, pl.C, pl.Kmax);
    void* bt_ws = with_tb ? cv.take<char>(tsm::backtrace_ws_bytes(btp, pl.B)) : nullptr;
    tsm::ScanParams p = scan_params(pl, w, cum, tr, db, len, ps, pe);
    p.emit = emit;
    p.val = nullptr;
    p.lvl = nullptr;
    p.zout = score;
    p.bp = bp;
    hipStream_t st = (hipStream_t)stream;
    // cooperative plans (C > 64): the max-plus cooperative scan, with backpointers
    int e = pl.fast ? tsm::launch_scan_viterbi(pl, p, st) : tsm::launch_scan_forward(pl, p, TSM_SEMIRING_MAX, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_viterbi (factorised scan)");
    if (with_tb) {
      e = tsm::launch_fact_to_exact(bp, len, pl.B, pl.T, pl.C, bp_exact, st);
      if (e != hipSuccess) return hip_fail(e, "tsm_viterbi (backpointer format)");
      e = tsm::launch_backtrace(btp, bp_exact, w.fin, nullptr, len, pl.B, pl.T, pl.C, pl.Kmax, bt_ws, seg_count,
                                segments, st);
      if (e != hipSuccess) return hip_fail(e, "tsm_viterbi (backtrace)");
    }
    return TSM_OK;
  }
  if (cum == nullptr) return fail(TSM_ERR_INVALID, "tsm_viterbi: the exact kernel needs cum_scores");
  const DeviceInfo di = device_info();
  const size_t lds = tsm::viterbi_lds_bytes(pl.C, pl.Kmax, pl.RS, ps != nullptr);
  if (lds > (size_t)di.max_lds)
    return fail(TSM_ERR_UNSUPPORTED, "Viterbi ring (C=%d, K=%d) needs %zu bytes of LDS (> %d)", pl.C, pl.K, lds,
                di.max_lds);
  const size_t need = viterbi_ws_bytes(pl, with_tb);
  if (!workspace || ws_bytes < need)
    return fail(TSM_ERR_WORKSPACE, "viterbi workspace too small: %zu < %zu bytes", ws_bytes, need);
  Carver cv(workspace);
  tsm::ViterbiParams v{};
  v.bp = with_tb ? cv.take<int32_t>((size_t)pl.B * (pl.T + 1) * pl.C) : nullptr;
  v.final_c = cv.take<int32_t>(pl.B);
  v.cum = cum;
  v.trans = tr;
  v.db = db;
  v.lengths = len;
  v.ps = ps;
  v.pe = pe;
  v.B = pl.B;
  v.T = pl.T;
  v.C = pl.C;
  v.K = pl.K;
  v.Kmax = pl.Kmax;
  v.RS = pl.RS;
  v.trows = pl.trows;
  v.score = score;
  void* bt_ws = nullptr;
  tsm::BtPlan btp{};
  if (with_tb) {
    btp = tsm::backtrace_plan(pl.B, pl.T, pl.C, pl.Kmax);
    bt_ws = cv.take<char>(tsm::backtrace_ws_bytes(btp, pl.B));
  }
  hipStream_t st = (hipStream_t)stream;
  int e = tsm::launch_viterbi(pl, v, st);
  if (e != hipSuccess) return hip_fail(e, "tsm_viterbi");
  if (with_tb) {
    e = tsm::launch_backtrace(btp, v.bp, nullptr, v.final_c, len, pl.B, pl.T, pl.C, pl.Kmax, bt_ws, seg_count,
                              segments, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_viterbi (backtrace)");
  }
  return TSM_OK;
}

}  // namespace

extern "C" {

int tsm_viterbi(const float* cum, const float* tr, const float* db, const int64_t* len, const float* ps,
                const float* pe, int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, float* score,
                int with_tb, int algorithm, int32_t* seg_count, int32_t* segments, void* workspace, size_t ws_bytes,
                void* stream) {
  if (!cum) return fail(TSM_ERR_INVALID, "cum_scores, transition, duration_bias and lengths are required");
  return viterbi_impl(cum, nullptr, tr, db, len, ps, pe, B, T, C, K, trans_rows, score, with_tb, algorithm,
                      seg_count, segments, workspace, ws_bytes, stream);
}

int tsm_segment_terms(const float* cum, const float* tr, const float* db, const int32_t* seg_count,
                      const int32_t* segments, int64_t B, int64_t T, int64_t C, int64_t K, double* out, void* stream) {
  if (!cum || !tr || !db || !seg_count || !segments || !out)
    return fail(TSM_ERR_INVALID, "cum_scores, transition, duration_bias, seg_count, segments and out are required");
  if (B < 0 || T < 0 || C < 1 || K < 1)
    return fail(TSM_ERR_INVALID, "need B, T >= 0 and C, K >= 1 (got %lld, %lld, %lld, %lld)", (long long)B,
                (long long)T, (long long)C, (long long)K);
  if (T >= (int64_t)1 << 30 || B > 65535 || C > 4096 || K > (int64_t)1 << 30)
    return fail(TSM_ERR_UNSUPPORTED, "segment terms: sizes too large (B=%lld, T=%lld, C=%lld)", (long long)B,
                (long long)T, (long long)C);
  const int e = tsm::launch_segment_terms(cum, tr, db, seg_count, segments, (int)B, (int)T, (int)C, (int)K, out,
                                          (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "tsm_segment_terms");
  return TSM_OK;
}

int tsm_prologue_workspace(int64_t B, int64_t T, int64_t C, size_t* bytes) {
  if (!bytes) return fail(TSM_ERR_INVALID, "bytes is NULL");
  if (B < 1 || T < 1 || C < 1)
    return fail(TSM_ERR_INVALID, "need B, T, C >= 1 (got %lld, %lld, %lld)", (long long)B, (long long)T, (long long)C);
  if (T > (int64_t)1 << 30 || B * C > (int64_t)1 << 30)
    return fail(TSM_ERR_UNSUPPORTED, "prologue: sizes too large (B=%lld, T=%lld, C=%lld)", (long long)B,
                (long long)T, (long long)C);
  const size_t nbl = (size_t)tsm::prologue_blocks((int)T);
  Carver cv(nullptr);
  cv.take<double>((size_t)B * nbl * C);
  cv.take<double>((size_t)B * nbl * C);
  cv.take<double>((size_t)B * C);
  *bytes = cv.off + 256;
  return TSM_OK;
}

static int run_prologue(const void* x, int dtype, const float* g, int64_t B, int64_t T, int64_t C, int centre,
                        float* cum, float* gx, void* workspace, size_t ws_bytes, void* stream, const char* what) {
  size_t need = 0;
  int rc = tsm_prologue_workspace(B, T, C, &need);
  if (rc) return rc;
  if (!workspace || ws_bytes < need)
    return fail(TSM_ERR_WORKSPACE, "%s: workspace too small: %zu < %zu bytes", what, ws_bytes, need);
  const size_t nbl = (size_t)tsm::prologue_blocks((int)T);
  Carver cv(workspace);
  tsm::PrologueParams q{};
  q.part = cv.take<double>((size_t)B * nbl * C);
  q.part2 = cv.take<double>((size_t)B * nbl * C);
  q.mean = cv.take<double>((size_t)B * C);
  q.x = x;
  q.dtype = dtype;
  q.g = g;
  q.cum = cum;
  q.gx = gx;
  q.B = (int)B;
  q.T = (int)T;
  q.C = (int)C;
  q.NBL = (int)nbl;
  q.centre = centre ? 1 : 0;
  q.GR = (int)T + 1;
  q.goff = 0;
  if (g != nullptr && g == gx) {  // the cum gradient held in grad_x itself, row u at row u-1
    q.GR = (int)T;
    q.goff = -1;
  }
  const int e = tsm::launch_prologue(q, g != nullptr, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, what);
  return TSM_OK;
}

int tsm_cum_scores(const void* scores, int dtype, int64_t B, int64_t T, int64_t C, int centre, float* cum,
                   void* workspace, size_t ws_bytes, void* stream) {
  if (!scores || !cum) return fail(TSM_ERR_INVALID, "scores and cum_scores are required");
  if (dtype != TSM_DTYPE_F32 && dtype != TSM_DTYPE_BF16 && dtype != TSM_DTYPE_F16)
    return fail(TSM_ERR_INVALID, "dtype must be TSM_DTYPE_F32 (0), _BF16 (1) or _F16 (2), got %d", dtype);
  return run_prologue(scores, dtype, nullptr, B, T, C, centre, cum, nullptr, workspace, ws_bytes, stream,
                      "tsm_cum_scores");
}

int tsm_cum_scores_backward(const float* grad_cum, int64_t B, int64_t T, int64_t C, int centre, float* grad_scores,
                            void* workspace, size_t ws_bytes, void* stream) {
  if (!grad_cum || !grad_scores) return fail(TSM_ERR_INVALID, "grad_cum and grad_scores are required");
  return run_prologue(nullptr, TSM_DTYPE_F32, grad_cum, B, T, C, centre, nullptr, grad_scores, workspace, ws_bytes,
                      stream, "tsm_cum_scores_backward");
}

int tsm_gold_score_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t db_rows, size_t* bytes) {
  if (!bytes) return fail(TSM_ERR_INVALID, "bytes is NULL");
  int rc = check_gold(B, T, C, K, db_rows);
  if (rc) return rc;
  Carver cv(nullptr);
  carve_gold(cv, B, T, C, db_rows);
  *bytes = cv.off + 256;
  return TSM_OK;
}

int tsm_gold_score(const float* cum, const float* tr, const float* db, const int64_t* labels, const int64_t* len,
                   int64_t B, int64_t T, int64_t C, int64_t K, int64_t db_rows, float* score, void* workspace,
                   size_t ws_bytes, void* stream) {
  if (!cum || !tr || !db || !labels || !len || !score)
    return fail(TSM_ERR_INVALID, "cum_scores, transition, duration_bias, labels, lengths and score are required");
  int rc = check_gold(B, T, C, K, db_rows);
  if (rc) return rc;
  size_t need = 0;
  tsm_gold_score_workspace(B, T, C, K, db_rows, &need);
  if (!workspace || ws_bytes < need)
    return fail(TSM_ERR_WORKSPACE, "gold score workspace too small: %zu < %zu bytes", ws_bytes, need);
  Carver cv(workspace);
  const GoldWs w = carve_gold(cv, B, T, C, db_rows);
  tsm::GoldParams g = gold_params(w, cum, tr, db, labels, len, B, T, C, K, db_rows);
  g.score = score;
  const int e = tsm::launch_gold_score(g, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "tsm_gold_score");
  return TSM_OK;
}

int tsm_gold_score_backward(const int64_t* labels, const int64_t* len, int64_t B, int64_t T, int64_t C, int64_t K,
                            int64_t db_rows, const float* grad_output, float* grad_cum, float* grad_tr,
                            float* grad_db, void* workspace, size_t ws_bytes, void* stream) {
  if (!labels || !len || !grad_output || !grad_cum || !grad_tr || !grad_db)
    return fail(TSM_ERR_INVALID, "labels, lengths, grad_output and the gradient outputs are required");
  int rc = check_gold(B, T, C, K, db_rows);
  if (rc) return rc;
  size_t need = 0;
  tsm_gold_score_workspace(B, T, C, K, db_rows, &need);
  if (!workspace || ws_bytes < need)
    return fail(TSM_ERR_WORKSPACE, "gold score workspace too small: %zu < %zu bytes", ws_bytes, need);
  Carver cv(workspace);
  const GoldWs w = carve_gold(cv, B, T, C, db_rows);
  tsm::GoldParams g = gold_params(w, nullptr, nullptr, nullptr, labels, len, B, T, C, K, db_rows);
  g.gout = grad_output;
  g.gcum = grad_cum;
  g.gtr = grad_tr;
  g.gdb = grad_db;
  const int e = tsm::launch_gold_backward(g, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "tsm_gold_score_backward");
  return TSM_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Emission input: the same passes on projected scores (B, T, C) instead of
// cumulative scores.  The register-resident scans and marginals (and the
// coverage passes) read the scores themselves and carry cum in registers, so
// no (B, T+1, C) cumulative tensor is built; a call whose plan runs other
// kernels (generic or cooperative scans, duration-dependent transitions, the
// exact Viterbi kernel) builds cum in its workspace with the prologue first.
// ---------------------------------------------------------------------------
namespace {

bool emit_fused_fwd(const Plan& pl, int semiring) {
  return semiring == TSM_SEMIRING_LOG && pl.fast && !pl.dense && pl.T >= 1;
}
bool emit_fused_bwd(const Plan& pl, int semiring) {
  return semiring == TSM_SEMIRING_LOG && pl.fast && !pl.dense && (pl.mfused || pl.mfast) && pl.T >= 1;
}

size_t prologue_bytes(const Plan& pl) {
  size_t n = 0;
  tsm_prologue_workspace(pl.B, pl.T, pl.C, &n);
  return n;
}

// workspace of the built-cum path: cum (B, T+1, C) and the prologue's scratch
size_t emit_cum_bytes(const Plan& pl) {
  Carver cv(nullptr);
  cv.take<float>((size_t)pl.B * (pl.T + 1) * pl.C);
  cv.take<char>(prologue_bytes(pl));
  return (cv.off + 255) & ~size_t(255);
}

// Builds cum from the scores at the start of the workspace; returns the rest.
int emit_build_cum(const Plan& pl, const float* scores, void* ws, size_t ws_bytes, void* stream, float** cum,
                   void** rest, size_t* rest_bytes, const char* what) {
  const size_t head = emit_cum_bytes(pl);
  if (!ws || ws_bytes < head) return fail(TSM_ERR_WORKSPACE, "%s: workspace too small: %zu < %zu bytes", what, ws_bytes, head);
  Carver cv(ws);
  *cum = cv.take<float>((size_t)pl.B * (pl.T + 1) * pl.C);
  const size_t pb = prologue_bytes(pl);
  void* pw = cv.take<char>(pb);
  const int rc = run_prologue(scores, TSM_DTYPE_F32, nullptr, pl.B, pl.T, pl.C, 0, *cum, nullptr, pw, pb, stream, what);
  if (rc) return rc;
  *rest = static_cast<char*>(ws) + head;
  *rest_bytes = ws_bytes - head;
  return TSM_OK;
}

int emit_plan(const float* scores, int64_t B, int64_t T, int64_t C, int64_t K, int has_ps, int has_pe,
              int64_t trans_rows, Plan* pl, const char* what) {
  if (!scores) return fail(TSM_ERR_INVALID, "%s: scores are required", what);
  if (T < 1) return fail(TSM_ERR_INVALID, "%s: scores need T >= 1 positions (got %lld)", what, (long long)T);
  return make_plan(B, T, C, K, has_ps, has_pe, trans_rows, pl);
}

}  // namespace

extern "C" {

int tsm_forward_emissions_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int semiring,
                                    int has_ps, int has_pe, size_t* bytes) {
  if (!bytes) return fail(TSM_ERR_INVALID, "bytes is NULL");
  if (semiring != TSM_SEMIRING_LOG && semiring != TSM_SEMIRING_MAX) return fail(TSM_ERR_INVALID, "bad semiring %d", semiring);
  if (T < 1) return fail(TSM_ERR_INVALID, "scores need T >= 1 positions (got %lld)", (long long)T);
  Plan p;
  const int rc = make_plan(B, T, C, K, has_ps, has_pe, trans_rows, &p);
  if (rc) return rc;
  *bytes = forward_ws_bytes(p, semiring) + (emit_fused_fwd(p, semiring) ? 0 : emit_cum_bytes(p));
  return TSM_OK;
}

int tsm_forward_emissions(const float* scores, const float* tr, const float* db, const int64_t* len, const float* ps,
                          const float* pe, int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows,
                          int semiring, float* partition, double* log2_partition, float* alpha_hat,
                          double* alpha_level, int32_t* recomputed, void* workspace, size_t ws_bytes, void* stream) {
  Plan pl;
  int rc = emit_plan(scores, B, T, C, K, ps != nullptr, pe != nullptr, trans_rows, &pl, "tsm_forward_emissions");
  if (rc) return rc;
  if (emit_fused_fwd(pl, semiring))
    return forward_impl(nullptr, tr, db, len, ps, pe, B, T, C, K, trans_rows, semiring, partition, log2_partition,
                        alpha_hat, alpha_level, recomputed, workspace, ws_bytes, stream, "tsm_forward_emissions",
                        scores);
  float* cum = nullptr;
  void* rest = nullptr;
  size_t rest_bytes = 0;
  rc = emit_build_cum(pl, scores, workspace, ws_bytes, stream, &cum, &rest, &rest_bytes, "tsm_forward_emissions");
  if (rc) return rc;
  return forward_impl(cum, tr, db, len, ps, pe, B, T, C, K, trans_rows, semiring, partition, log2_partition,
                      alpha_hat, alpha_level, recomputed, rest, rest_bytes, stream, "tsm_forward_emissions");
}

int tsm_backward_emissions_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int semiring,
                                     int has_ps, int has_pe, size_t* bytes) {
  if (!bytes) return fail(TSM_ERR_INVALID, "bytes is NULL");
  if (semiring != TSM_SEMIRING_LOG && semiring != TSM_SEMIRING_MAX) return fail(TSM_ERR_INVALID, "bad semiring %d", semiring);
  if (T < 1) return fail(TSM_ERR_INVALID, "scores need T >= 1 positions (got %lld)", (long long)T);
  Plan p;
  const int rc = make_plan(B, T, C, K, has_ps, has_pe, trans_rows, &p);
  if (rc) return rc;
  const size_t tail = (backward_ws_bytes(p) + 255) & ~size_t(255);
  if (emit_fused_bwd(p, semiring)) {
    *bytes = tail + prologue_bytes(p);
  } else {
    // cum and its prologue scratch, the cum gradient, the backward's own workspace
    *bytes = emit_cum_bytes(p) + (((size_t)p.B * (p.T + 1) * p.C * 4 + 255) & ~size_t(255)) + tail;
  }
  return TSM_OK;
}

int tsm_backward_emissions(const float* scores, const float* tr, const float* db, const int64_t* len,
                           const float* ps, const float* pe, int64_t B, int64_t T, int64_t C, int64_t K,
                           int64_t trans_rows, int semiring, const float* alpha_hat, const double* alpha_level,
                           const double* log2_partition, const float* grad_output, float* grad_scores,
                           float* grad_tr, float* grad_db, float* grad_ps, float* grad_pe, int32_t* recomputed,
                           void* workspace, size_t ws_bytes, void* stream) {
  Plan pl;
  int rc = emit_plan(scores, B, T, C, K, ps != nullptr, pe != nullptr, trans_rows, &pl, "tsm_backward_emissions");
  if (rc) return rc;
  if (!grad_scores) return fail(TSM_ERR_INVALID, "tsm_backward_emissions: grad_scores is required");
  size_t need = 0;
  rc = tsm_backward_emissions_workspace(B, T, C, K, trans_rows, semiring, ps != nullptr, pe != nullptr, &need);
  if (rc) return rc;
  if (!workspace || ws_bytes < need)
    return fail(TSM_ERR_WORKSPACE, "tsm_backward_emissions: workspace too small: %zu < %zu bytes", ws_bytes, need);
  if (emit_fused_bwd(pl, semiring)) {
    // the kernels read the scores; the finalize leaves row t >= 1 of the cum gradient
    // at row t-1 of grad_scores, and the suffix sums run in place there
    const size_t tail = (backward_ws_bytes(pl) + 255) & ~size_t(255);
    rc = backward_impl(nullptr, scores, tr, db, len, ps, pe, B, T, C, K, trans_rows, semiring, alpha_hat,
                       alpha_level, log2_partition, grad_output, grad_scores, grad_tr, grad_db, grad_ps, grad_pe,
                       recomputed, workspace, tail, stream);
    if (rc) return rc;
    return run_prologue(nullptr, TSM_DTYPE_F32, grad_scores, B, T, C, 0, nullptr, grad_scores,
                        static_cast<char*>(workspace) + tail, ws_bytes - tail, stream,
                        "tsm_backward_emissions (score gradient)");
  }
  float* cum = nullptr;
  void* rest = nullptr;
  size_t rest_bytes = 0;
  rc = emit_build_cum(pl, scores, workspace, ws_bytes, stream, &cum, &rest, &rest_bytes, "tsm_backward_emissions");
  if (rc) return rc;
  const size_t gbytes = ((size_t)pl.B * (pl.T + 1) * pl.C * 4 + 255) & ~size_t(255);
  float* gcum = static_cast<float*>(rest);
  rc = backward_impl(cum, nullptr, tr, db, len, ps, pe, B, T, C, K, trans_rows, semiring, alpha_hat, alpha_level,
                     log2_partition, grad_output, gcum, grad_tr, grad_db, grad_ps, grad_pe, recomputed,
                     static_cast<char*>(rest) + gbytes, rest_bytes - gbytes, stream);
  if (rc) return rc;
  // the prologue's scratch (in the cum head of the workspace) is free again
  Carver cv(workspace);
  cv.take<float>((size_t)pl.B * (pl.T + 1) * pl.C);
  void* pw = cv.take<char>(prologue_bytes(pl));
  return run_prologue(nullptr, TSM_DTYPE_F32, gcum, B, T, C, 0, nullptr, grad_scores, pw, prologue_bytes(pl), stream,
                      "tsm_backward_emissions (score gradient)");
}

int tsm_viterbi_emissions_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int with_tb,
                                    int algorithm, size_t* bytes) {
  if (!bytes) return fail(TSM_ERR_INVALID, "bytes is NULL");
  if (T < 1) return fail(TSM_ERR_INVALID, "scores need T >= 1 positions (got %lld)", (long long)T);
  Plan p;
  const int rc = make_plan(B, T, C, K, 0, 0, trans_rows, &p);
  if (rc) return rc;
  // (the register-resident scans read the scores; every other kernel reads cum_scores built first)
  *bytes = viterbi_ws_bytes(p, with_tb) + ((viterbi_factorised(p, algorithm) && p.fast) ? 0 : emit_cum_bytes(p));
  return TSM_OK;
}

int tsm_viterbi_emissions(const float* scores, const float* tr, const float* db, const int64_t* len,
                          const float* ps, const float* pe, int64_t B, int64_t T, int64_t C, int64_t K,
                          int64_t trans_rows, float* score, int with_tb, int algorithm, int32_t* seg_count,
                          int32_t* segments, void* workspace, size_t ws_bytes, void* stream) {
  Plan pl;
  int rc = emit_plan(scores, B, T, C, K, ps != nullptr, pe != nullptr, trans_rows, &pl, "tsm_viterbi_emissions");
  if (rc) return rc;
  if (algorithm < TSM_VITERBI_AUTO || algorithm > TSM_VITERBI_FACTORISED)
    return fail(TSM_ERR_INVALID, "algorithm must be TSM_VITERBI_AUTO (0), _EXACT (1) or _FACTORISED (2), got %d",
                algorithm);
  if (viterbi_factorised(pl, algorithm) && pl.fast)
    return viterbi_impl(nullptr, scores, tr, db, len, ps, pe, B, T, C, K, trans_rows, score, with_tb, algorithm,
                        seg_count, segments, workspace, ws_bytes, stream);
  float* cum = nullptr;
  void* rest = nullptr;
  size_t rest_bytes = 0;
  rc = emit_build_cum(pl, scores, workspace, ws_bytes, stream, &cum, &rest, &rest_bytes, "tsm_viterbi_emissions");
  if (rc) return rc;
  return viterbi_impl(cum, nullptr, tr, db, len, ps, pe, B, T, C, K, trans_rows, score, with_tb, algorithm,
                      seg_count, segments, rest, rest_bytes, stream);
}

int tsm_gold_score_emissions(const float* scores, const float* tr, const float* db, const int64_t* labels,
                             const int64_t* len, int64_t B, int64_t T, int64_t C, int64_t K, int64_t db_rows,
                             float* score, void* workspace, size_t ws_bytes, void* stream) {
  if (!scores || !tr || !db || !labels || !len || !score)
    return fail(TSM_ERR_INVALID, "scores, transition, duration_bias, labels, lengths and score are required");
  int rc = check_gold(B, T, C, K, db_rows);
  if (rc) return rc;
  size_t need = 0;
  tsm_gold_score_workspace(B, T, C, K, db_rows, &need);
  if (!workspace || ws_bytes < need)
    return fail(TSM_ERR_WORKSPACE, "gold score workspace too small: %zu < %zu bytes", ws_bytes, need);
  Carver cv(workspace);
  const GoldWs w = carve_gold(cv, B, T, C, db_rows);
  tsm::GoldParams g = gold_params(w, nullptr, tr, db, labels, len, B, T, C, K, db_rows);
  g.emit = scores;
  g.score = score;
  const int e = tsm::launch_gold_score(g, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "tsm_gold_score_emissions");
  return TSM_OK;
}

int tsm_gold_score_emissions_backward(const int64_t* labels, const int64_t* len, int64_t B, int64_t T, int64_t C,
                                      int64_t K, int64_t db_rows, const float* grad_output, float* grad_scores,
                                      float* grad_tr, float* grad_db, void* workspace, size_t ws_bytes,
                                      void* stream) {
  if (!labels || !len || !grad_output || !grad_scores || !grad_tr || !grad_db)
    return fail(TSM_ERR_INVALID, "labels, lengths, grad_output and the gradient outputs are required");
  int rc = check_gold(B, T, C, K, db_rows);
  if (rc) return rc;
  size_t need = 0;
  tsm_gold_score_workspace(B, T, C, K, db_rows, &need);
  if (!workspace || ws_bytes < need)
    return fail(TSM_ERR_WORKSPACE, "gold score workspace too small: %zu < %zu bytes", ws_bytes, need);
  Carver cv(workspace);
  const GoldWs w = carve_gold(cv, B, T, C, db_rows);
  tsm::GoldParams g = gold_params(w, nullptr, nullptr, nullptr, labels, len, B, T, C, K, db_rows);
  g.gout = grad_output;
  g.gcum = grad_scores;
  g.emit_grad = 1;
  g.gtr = grad_tr;
  g.gdb = grad_db;
  const int e = tsm::launch_gold_backward(g, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "tsm_gold_score_emissions_backward");
  return TSM_OK;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Bounded-memory (checkpointed) forward and backward.  The forward keeps no
// alpha table: only, per window start (windows of whole chunks), the ring
// state that the chunk ending there recorded and the alpha-hat row there.  The
// backward runs each window as a problem of its own, top window first: the
// forward over the window from its start state (alpha-hat for one window),
// then the fused backward from the state that the window above recorded at its
// position 0; rows at window edges add up across windows.  Memory: one
// window's tables instead of the whole sequence's.  Reference counterpart:
// the ring checkpoints and per-segment alpha recomputation of
// streaming/pytorch_reference.py:380-423.
// ---------------------------------------------------------------------------
namespace {

int ck_plan(int64_t B, int64_t T, int64_t C, int64_t K, int has_ps, int has_pe, Plan* pl) {
  const int rc = make_plan(B, T, C, K, has_ps, has_pe, 0, pl, 16);
  if (rc) return rc;
  if (!pl->fast || pl->FJ != 16 || !pl->mfused)
    return fail(TSM_ERR_UNSUPPORTED,
                "the bounded-memory backward runs the 16-lane register-resident scans with fused marginals "
                "(C <= 64, K <= 513, static transitions); this problem has no such plan");
  return TSM_OK;
}

// One window's buffers: alpha-hat and levels, scratch outputs of its forward,
// the forward's scan workspace and the backward's workspace.
struct WinWs {
  float* ah;
  double* al;
  double* z2;
  float* zout;
  ScanWs fs;
  BwdWs bw;
};

WinWs carve_window(Carver& cv, const Plan& pw) {
  WinWs w;
  w.ah = cv.take<float>((size_t)pw.B * (pw.T + 1) * pw.C);
  w.al = cv.take<double>((size_t)pw.B * (pw.T + 1));
  w.z2 = cv.take<double>((size_t)pw.B);
  w.zout = cv.take<float>((size_t)pw.B);
  w.fs = carve_scan(cv, pw, false);
  w.bw = carve_backward(cv, pw);
  return w;
}

struct CkGeom {
  Plan full, win, last;
  int Wlen = 0, nw = 0;
};

// Fixed part of the backward workspace (per-window lengths and flags, the
// states handed between windows, the end sums beyond a window) and the window
// region (the larger of a full and the last window).
struct CkFixed {
  int64_t* lenw;
  int *okf, *okb;
  float *st[2], *thalo;
  double* lv[2];
};

CkFixed carve_ck_fixed(Carver& cv, const CkGeom& g) {
  CkFixed f;
  const size_t n = (size_t)g.full.B * g.nw;
  const size_t KC = (size_t)g.full.B * g.full.Kmax * g.full.C;
  f.lenw = cv.take<int64_t>(n);
  f.okf = cv.take<int>(n);
  f.okb = cv.take<int>(n);
  for (int i = 0; i < 2; ++i) {
    f.st[i] = cv.take<float>(KC);
    f.lv[i] = cv.take<double>((size_t)g.full.B * g.full.Kmax);
  }
  f.thalo = cv.take<float>(KC);
  return f;
}

size_t ck_backward_bytes(const CkGeom& g) {
  Carver cf(nullptr);
  carve_ck_fixed(cf, g);
  const size_t fixed = (cf.off + 255) & ~size_t(255);
  Carver a(nullptr), b(nullptr);
  carve_window(a, g.win);
  carve_window(b, g.last);
  return fixed + std::max(a.off, b.off) + 256;
}

int ck_window_plans(CkGeom& g, int has_ps, int has_pe) {
  const int64_t T = g.full.T, B = g.full.B;
  int rc = ck_plan(B, std::min<int64_t>(g.Wlen, T), g.full.C, g.full.K, has_ps, has_pe, &g.win);
  if (rc) return rc;
  const int64_t last = T - (int64_t)(g.nw - 1) * g.Wlen;
  return ck_plan(B, last, g.full.C, g.full.K, has_ps, has_pe, &g.last);
}

int ck_geometry(int64_t B, int64_t T, int64_t C, int64_t K, int has_ps, int has_pe, int64_t window, CkGeom* g) {
  int rc = ck_plan(B, T, C, K, has_ps, has_pe, &g->full);
  if (rc) return rc;
  const int Lc = g->full.Lc;
  if (window < Lc || window % Lc != 0)
    return fail(TSM_ERR_INVALID, "window must be a positive multiple of the chunk length %d (got %lld)", Lc,
                (long long)window);
  g->Wlen = (int)std::min<int64_t>(window, (int64_t)cdiv(T, Lc) * Lc);
  g->nw = (int)cdiv(T, g->Wlen);
  return ck_window_plans(*g, has_ps, has_pe);
}

}  // namespace

extern "C" {

int tsm_checkpoint_plan(int64_t B, int64_t T, int64_t C, int64_t K, int has_ps, int has_pe, size_t budget_bytes,
                        int64_t* window, int64_t* n_windows, size_t* forward_ws, size_t* backward_ws) {
  if (!window || !n_windows || !forward_ws || !backward_ws) return fail(TSM_ERR_INVALID, "null output pointer");
  CkGeom g;
  int rc = ck_plan(B, T, C, K, has_ps, has_pe, &g.full);
  if (rc) return rc;
  const int Lc = g.full.Lc, P = (int)cdiv(T, Lc);
  // the longest window of whole chunks whose backward workspace fits the budget
  // (budget 0: about eight windows)
  int best = 1;
  if (budget_bytes == 0) {
    best = std::max(1, (int)cdiv(P, 8));
  } else {
    for (int wc = P; wc >= 1; wc = (wc > 8 ? wc - (wc + 7) / 8 : wc - 1)) {
      CkGeom h = g;
      h.Wlen = wc * Lc;
      h.nw = (int)cdiv(T, h.Wlen);
      if (ck_window_plans(h, has_ps, has_pe)) return TSM_ERR_UNSUPPORTED;
      if (ck_backward_bytes(h) <= budget_bytes) {
        best = wc;
        break;
      }
    }
  }
  rc = ck_geometry(B, T, C, K, has_ps, has_pe, (int64_t)best * Lc, &g);
  if (rc) return rc;
  *window = g.Wlen;
  *n_windows = g.nw;
  Carver cv(nullptr);
  carve_scan(cv, g.full, false);
  *forward_ws = cv.off + 256;
  *backward_ws = ck_backward_bytes(g);
  return TSM_OK;
}

int tsm_checkpointed_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int has_ps, int has_pe, int64_t window,
                               size_t* forward_ws, size_t* backward_ws) {
  if (!forward_ws || !backward_ws) return fail(TSM_ERR_INVALID, "null output pointer");
  CkGeom g;
  const int rc = ck_geometry(B, T, C, K, has_ps, has_pe, window, &g);
  if (rc) return rc;
  Carver cv(nullptr);
  carve_scan(cv, g.full, false);
  *forward_ws = cv.off + 256;
  *backward_ws = ck_backward_bytes(g);
  return TSM_OK;
}

int tsm_forward_checkpointed(const float* cum, const float* tr, const float* db, const int64_t* len, const float* ps,
                             const float* pe, int64_t B, int64_t T, int64_t C, int64_t K, int64_t window,
                             float* partition, double* log2_partition, float* ck_state, double* ck_level,
                             float* ck_alpha, double* ck_alpha_level, void* workspace, size_t ws_bytes,
                             void* stream) {
  int rc = check_common(cum, tr, db, len, TSM_SEMIRING_LOG);
  if (rc) return rc;
  if (!partition || !ck_state || !ck_level || !ck_alpha || !ck_alpha_level)
    return fail(TSM_ERR_INVALID, "partition and the checkpoint outputs are required");
  CkGeom g;
  rc = ck_geometry(B, T, C, K, ps != nullptr, pe != nullptr, window, &g);
  if (rc) return rc;
  Carver need(nullptr);
  carve_scan(need, g.full, false);
  if (!workspace || ws_bytes < need.off + 256)
    return fail(TSM_ERR_WORKSPACE, "tsm_forward_checkpointed: workspace too small: %zu < %zu bytes", ws_bytes,
                need.off + 256);
  hipStream_t st = (hipStream_t)stream;
  Carver cv(workspace);
  ScanWs w = carve_scan(cv, g.full, false);
  tsm::ScanParams p = scan_params(g.full, w, cum, tr, db, len, ps, pe);
  p.win = 1;
  p.xseq = (T + 1) * C;
  p.pseq = T * C;
  p.val = nullptr;
  p.lvl = nullptr;
  if (log2_partition) p.z2 = log2_partition;
  p.zout = partition;
  p.ck_ah = ck_alpha;
  p.ck_al = ck_alpha_level;
  p.ck_every = g.Wlen;
  p.ck_n = g.nw;
  int e = tsm::launch_scan_forward(g.full, p, TSM_SEMIRING_LOG, st);
  if (e != hipSuccess) return hip_fail(e, "tsm_forward_checkpointed");
  e = tsm::launch_ck_extract(w.st_end, w.lv_end, w.offs, g.full.B, g.full.P, g.Wlen / g.full.Lc, g.full.Kmax, g.full.C,
                             g.nw, ck_state, ck_level, ck_alpha_level, st);
  if (e != hipSuccess) return hip_fail(e, "tsm_forward_checkpointed (checkpoints)");
  return TSM_OK;
}

int tsm_backward_checkpointed(const float* cum, const float* tr, const float* db, const int64_t* len,
                              const float* ps, const float* pe, int64_t B, int64_t T, int64_t C, int64_t K,
                              int64_t window, const float* ck_state, const double* ck_level, const float* ck_alpha,
                              const double* ck_alpha_level, const double* log2_partition, const float* grad_output,
                              float* grad_cum, float* grad_tr, float* grad_db, float* grad_ps, float* grad_pe,
                              void* workspace, size_t ws_bytes, void* stream) {
  int rc = check_common(cum, tr, db, len, TSM_SEMIRING_LOG);
  if (rc) return rc;
  if (!ck_state || !ck_level || !ck_alpha || !ck_alpha_level || !log2_partition || !grad_output || !grad_cum ||
      !grad_tr || !grad_db)
    return fail(TSM_ERR_INVALID, "the checkpoints, log2_partition, grad_output and the gradient outputs are required");
  if ((ps != nullptr) != (grad_ps != nullptr) || (pe != nullptr) != (grad_pe != nullptr))
    return fail(TSM_ERR_INVALID, "a projection gradient buffer is needed exactly when the projection is given");
  CkGeom g;
  rc = ck_geometry(B, T, C, K, ps != nullptr, pe != nullptr, window, &g);
  if (rc) return rc;
  const size_t need = ck_backward_bytes(g);
  if (!workspace || ws_bytes < need)
    return fail(TSM_ERR_WORKSPACE, "tsm_backward_checkpointed: workspace too small: %zu < %zu bytes", ws_bytes, need);
  hipStream_t st = (hipStream_t)stream;
  const int Kmax = g.full.Kmax;
  const size_t KC = (size_t)Kmax * C;
  // the outputs accumulate over windows
  int e = tsm::launch_fill_zero(grad_cum, (size_t)B * (T + 1) * C, st);
  if (e == hipSuccess) e = tsm::launch_fill_zero(grad_tr, (size_t)C * C, st);
  if (e == hipSuccess) e = tsm::launch_fill_zero(grad_db, (size_t)K * C, st);
  if (e == hipSuccess) e = tsm::launch_fill_zero(grad_ps, grad_ps ? (size_t)B * T * C : 0, st);
  if (e == hipSuccess) e = tsm::launch_fill_zero(grad_pe, grad_pe ? (size_t)B * T * C : 0, st);
  if (e != hipSuccess) return hip_fail(e, "tsm_backward_checkpointed (zero outputs)");
  Carver cv(workspace);
  const CkFixed fx = carve_ck_fixed(cv, g);
  char* region = static_cast<char*>(workspace) + ((cv.off + 255) & ~size_t(255));
  e = tsm::launch_window_setup(len, (int)B, (int)T, g.Wlen, g.nw, fx.lenw, fx.okf, fx.okb, st);
  if (e != hipSuccess) return hip_fail(e, "tsm_backward_checkpointed (windows)");
  const int64_t xseq = (T + 1) * C, pseq = T * C;
  int cur = 0;
  for (int w = g.nw - 1; w >= 0; --w) {
    // window w of every sequence: rows a .. a + Tw
    const Plan& pw = (w == g.nw - 1) ? g.last : g.win;
    const int64_t a = (int64_t)w * g.Wlen, Tw = pw.T;
    const size_t o = (size_t)w * B;  // the window's (B,) slice of lengths and flags
    Carver wc(region);
    const WinWs ww = carve_window(wc, pw);
    const float* cum_w = cum + a * C;
    const float* ps_w = ps ? ps + a * C : nullptr;
    const float* pe_w = pe ? pe + a * C : nullptr;
    // alpha over the window, from the forward's checkpoints at its start
    e = tsm::launch_window_row0(ck_alpha + o * C, ck_alpha_level + o, fx.okf + o, (int)B, (int)Tw, (int)C, ww.ah,
                                ww.al, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_backward_checkpointed (window start)");
    tsm::ScanParams p = scan_params(pw, ww.fs, cum_w, tr, db, fx.lenw + o, ps_w, pe_w);
    p.win = 1;
    p.xseq = xseq;
    p.pseq = pseq;
    p.org_st = ck_state + o * KC;
    p.org_lv = ck_level + o * Kmax;
    p.org_ok = fx.okf + o;
    p.val = ww.ah;
    p.lvl = ww.al;
    p.z2 = ww.z2;
    p.zout = ww.zout;
    e = tsm::launch_scan_forward(pw, p, TSM_SEMIRING_LOG, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_backward_checkpointed (window forward)");
    // the fused backward over the window, from the states the window above recorded
    const BwdWs& bw = ww.bw;
    tsm::FusedParams f{};
    f.lengths = fx.lenw + o;
    f.trans = tr;
    f.aval = ww.ah;
    f.uval = bw.uval;
    f.B = (int)B;
    f.T = (int)Tw;
    f.C = (int)C;
    f.K = pw.K;
    f.Kmax = Kmax;
    f.P = pw.P;
    f.Lc = pw.Lc;
    f.GNB = pw.GNB;
    f.GTB = pw.GTB;
    f.offs = bw.scan.offs;
    f.mframe = bw.mframe;
    f.cum = cum_w;
    f.db = db;
    f.ps = ps_w;
    f.alvl = ww.al;
    f.z2 = log2_partition;
    f.st_end = bw.scan.st_end;
    f.lv_end = bw.scan.lv_end;
    f.e_own = bw.e_own;
    f.s_out = bw.s_out;
    f.halo = bw.halo;
    f.db_part = bw.db_part;
    f.tr_part = bw.tr_part;
    f.grad_output = grad_output;
    f.grad_cum = grad_cum + a * C;
    f.grad_ps = grad_ps ? grad_ps + a * C : nullptr;
    f.grad_pe = grad_pe ? grad_pe + a * C : nullptr;
    f.grad_tr = grad_tr;
    f.grad_db = grad_db;
    f.accum = 1;
    f.org_ok = fx.okf + o;
    f.end_ok = fx.okb + o;
    f.xseq = xseq;
    f.pseq = pseq;
    e = tsm::launch_u_rows(pw, f, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_backward_checkpointed (u rows)");
    tsm::ScanParams q = scan_params(pw, bw.scan, cum_w, tr, db, fx.lenw + o, ps_w, pe_w);
    q.win = 1;
    q.xseq = xseq;
    q.pseq = pseq;
    q.org_st = fx.st[cur];
    q.org_lv = fx.lv[cur];
    q.org_ok = fx.okb + o;
    q.thalo = fx.thalo;
    // (no window below window 0: nothing to record, and no row before its position 0)
    q.tst_st = w >= 1 ? fx.st[1 - cur] : nullptr;
    q.tst_lv = w >= 1 ? fx.lv[1 - cur] : nullptr;
    q.val = nullptr;
    q.lvl = nullptr;
    q.zout = nullptr;
    q.uval = bw.uval;
    q.aval = ww.ah;
    q.alvl = ww.al;
    q.mz2 = log2_partition;
    q.e_own = bw.e_own;
    q.s_out = bw.s_out;
    q.halo = bw.halo;
    q.db_part = bw.db_part;
    q.mframe = bw.mframe;
    e = tsm::launch_scan_backward_fused(pw, q, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_backward_checkpointed (window beta scan)");
    e = tsm::launch_fused_finalize(pw, f, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_backward_checkpointed (window finalize)");
    if (w >= 1) e = tsm::launch_window_state_fix(fx.lv[1 - cur], bw.scan.offs, (int)B, pw.P, Kmax, st);
    if (e == hipSuccess)
      e = tsm::launch_window_halo_add(fx.thalo, bw.halo, bw.mframe, fx.lenw + o, fx.okb + o, (int)B, pw.P, pw.Lc, Kmax,
                                      (int)C, (int)(T - (a + Tw)), grad_output, grad_cum + (a + Tw) * C,
                                      grad_pe ? grad_pe + (a + Tw) * C : nullptr, xseq, pseq, st);
    if (e != hipSuccess) return hip_fail(e, "tsm_backward_checkpointed (window edges)");
    cur = 1 - cur;
  }
  return TSM_OK;
}

int tsm_ring_checkpoints(const float* alpha_hat, const double* alpha_level, const int64_t* len, int64_t B,
                         int64_t T, int64_t C, int64_t K, int64_t S, int64_t n_ckpt, float* out, void* stream) {
  if (!alpha_hat || !alpha_level || !len || !out) return fail(TSM_ERR_INVALID, "null pointer argument");
  if (B < 1 || T < 1 || C < 1 || K < 1 || S < 1 || n_ckpt < 0) return fail(TSM_ERR_INVALID, "bad sizes");
  if (n_ckpt == 0) return TSM_OK;
  const int e = tsm::launch_checkpoints(alpha_hat, alpha_level, len, (int)B, (int)T, (int)C, (int)K, (int)S,
                                        (int)n_ckpt, out, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "tsm_ring_checkpoints");
  return TSM_OK;
}

int tsm_timing_enable(int enable) {
  const int e = tsm::timing_enable(enable);
  if (e != hipSuccess) return hip_fail(e, "tsm_timing_enable");
  return TSM_OK;
}

int tsm_timing_read(double* total_ms, int64_t* launches, int n) {
  if (n < 0) return fail(TSM_ERR_INVALID, "n < 0");
  const int e = tsm::timing_read(total_ms, launches, n);
  if (e != hipSuccess) return hip_fail(e, "tsm_timing_read");
  return TSM_OK;
}

int tsm_timing_kernel_count(void) { return tsm::kNumKernels; }

const char* tsm_timing_kernel_name(int kernel_id) { return tsm::timing_name(kernel_id); }

}  // extern "C"
