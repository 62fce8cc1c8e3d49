// Kernel parameter blocks and host-side launchers (internal to libtsm_hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "tsm_plan.hpp"

namespace tsm {

enum Semiring : int { kLog = 0, kMax = 1 };

// Forward / backward chunked scan over one direction of the recursion.
struct ScanParams {
  // problem
  const float* cum;        // (B, T+1, C)
  const float* trans;      // (C, C)  transition[c_src][c_dst], natural log units
  const float* db;         // (K, C)  duration bias
  const int64_t* lengths;  // (B,)
  const float* ps;         // (B, T, C) proj_start or null
  const float* pe;         // (B, T, C) proj_end or null
  int B, T, C, K, Kmax, RS;
  int R, KP, RL;           // durations per lane, padded durations, ring row length
  int SB;                  // fused-marginal beta scan: steps per operand batch (power of two)
  int P, Lc, W;            // chunks per sequence, chunk length, warm-up
  int retry;               // 1: recompute only speculative chunks that failed verification
  float tol;               // verification tolerance, log2 units
  // per-position output (normalised log2 values and fp64 levels), may be null
  float* val;              // (B, T+1, C)
  double* lvl;             // (B, T+1)
  // chunk boundary states
  float* st_spec;          // (B*P, Kmax, C)
  double* lv_spec;         // (B*P, Kmax)
  float* st_end;           // (B*P, Kmax, C)
  double* lv_end;          // (B*P, Kmax)
  double* offs;            // (B*P) frame offsets (log2 units)
  double* vstat;           // (B*P, 2) max / min of exact - speculative boundary state
  int* status;             // (B*P) 0 exact, 1 speculative+verified, 2 recomputed
  int* vflag;              // set when the retry pass reran a chunk (the second verification is skipped otherwise)
  int* query_regs;         // plan time: the launch stores its scan kernel's VGPR count here and launches nothing
  int32_t* recomputed;     // (B) number of recomputed chunks, or null
  // forward only: final row at position len, partition
  float* fin;              // (B, C)
  double* fin_lvl;         // (B)
  double* z2;              // (B) log2 partition
  float* zout;             // (B) partition in natural log units
  // rings in global memory when LDS is too small
  float* gring;            // (B*P, scan_gring_floats)
  // max-semiring forward of the register-resident scan: per (b, t, c) the best
  // duration k of a segment ending at t and the best source label c' of a
  // segment starting at t, packed (k << 16 | c'); null otherwise
  int32_t* bp;
  // duration-dependent transitions (dense scans): number of transition
  // matrices (0: one static matrix) and the log2-scaled table of the scan's
  // direction, [k-1][out label][in label] for k = 1..Kmax
  int trows;
  const float* trx;
  // cooperative scan: G blocks per group, CL labels per block, NQ groups,
  // xmap = 1 when members share blockIdx % 8; per-group exchange buffers
  // (NQ, 2, C) of (fp32 value | step stamp) words and the give-up flag
  int G, CL, NQ, xmap;
  unsigned long long* xch;
  int* xabort;
  // backward scan with fused marginals: forward-side inputs and, per chunk
  // item (b*P + j), outputs in the chunk's frame (rescaled by the finalize)
  const float* uval;       // (B, T+1, C) u[t,c] = log2 sum_c' 2^(alpha-hat[t,c'] + trans[c',c] log2(e))
  const float* aval;       // (B, T+1, C) alpha-hat (log2)
  const double* alvl;      // (B, T+1) alpha levels
  const double* mz2;       // (B) log2 partition
  float* e_own;            // (B, T+1, C) end sums of the rows a chunk owns
  float* s_out;            // (B, T+1, C) start sums
  float* halo;             // (B*P, Kmax, C) end sums of rows t_hi .. t_hi+Kmax-1 of chunk j < jl
  double* db_part;         // (B*P, Kmax, C) duration sums
  double* mframe;          // (B*P) the chunk's frame estimate fr (log2)
  // emission input: (B, T, C) projected scores in place of cum (register-resident scans), or null
  const float* emit;
  // bounded-memory backward (win = 1: the problem is one window of longer
  // sequences; 16-lane log-semiring instances).  cum / ps / pe point at the
  // window's first row of sequence 0 and sequence b's rows start xseq / pseq
  // elements further (the full tensors' strides).  Chunks that would start
  // exactly from the sequence start / end start from org_st / org_lv (B, Kmax,
  // C) / (B, Kmax), ring format, global levels, where org_ok[b]; the forward
  // records alpha-hat rows t % ck_every == 0 in ck_ah (ck_n, B, C) / ck_al
  // (ck_n, B); the fused backward's top chunk writes the end sums of positions
  // len+1 .. len+Kmax-1 to thalo (B, Kmax, C), its chunk 0 its state at
  // position 0 to tst_st / tst_lv (chunk frame).
  int win;
  const float* org_st;
  const double* org_lv;
  const int* org_ok;
  float* ck_ah;
  double* ck_al;
  int ck_every, ck_n;
  float* thalo;
  float* tst_st;
  double* tst_lv;
  int64_t xseq, pseq;
};

struct MargParams {
  const float* cum;
  const float* emit;       // (B, T, C) projected scores in place of cum, or null
  const float* trans;
  const float* db;
  const int64_t* lengths;
  const float* ps;
  const float* pe;
  int B, T, C, K, Kmax, RS;
  int RL;                  // ring row length of the register-resident marginal kernel
  int NB, TB, CB, NCB;
  const float* aval;       // (B, T+1, C) alpha-hat (log2)
  const double* alvl;      // (B, T+1) alpha levels (global frame)
  const float* bval;       // (B, T+1, C) beta-hat (log2)
  const double* blvl;      // (B, T+1) beta levels (global frame)
  const double* z2;        // (B) log2 partition
  float* e_own;            // (B, T+1, C) end sums from starts inside the owning block
  float* s_out;            // (B, T+1, C) start sums
  float* halo;             // (B, NB, Kmax, C) end sums spilling into the next block
  double* db_part;         // (B, NB, Kmax, C)  duration-bias gradient partials
  double* tr_part;         // (B, NB, C, C)     transition gradient partials [c_src][c_dst]
                           // (B, NB, Kmax, C, C) with duration-dependent transitions
  int trows;               // number of transition matrices (0: one static matrix)
  const float* trx;        // dense: log2-scaled transitions [k-1][c_dst][c_src]
};

struct FinalParams {
  const int64_t* lengths;
  int B, T, C, K, Kmax, NB, TB;
  const float* e_own;
  const float* s_out;
  const float* halo;
  const double* db_part;
  const double* tr_part;
  const float* grad_output;  // (B)
  float* grad_cum;           // (B, T+1, C)
  float* grad_ps;            // (B, T, C) or null
  float* grad_pe;            // (B, T, C) or null
  float* grad_tr;            // (C, C)
  float* grad_db;            // (K, C)
  int trows;                 // grad_tr is (trows, C, C) when > 0
  const double* bscale;      // (B, NB) block scales of the coverage pass, or null (1)
  int shift;                 // 1: grad_cum is (B, T, C) and row t >= 1 goes to row t-1 (row 0 is dropped)
};

// Row passes of the backward with fused marginals (tsm_fused.hip).
struct FusedParams {
  const int64_t* lengths;
  const float* trans;      // (C, C) natural log units
  const float* aval;       // (B, T+1, C) alpha-hat
  float* uval;             // (B, T+1, C) written by the u pass
  int B, T, C, K, Kmax;
  int P, Lc;               // backward scan chunks per sequence, chunk length
  int GNB, GTB;            // transition-gradient row blocks per sequence, rows per block
  const double* offs;      // (B*P) verified level offsets of the backward chunks
  double* mframe;          // (B*P) frame estimates; the frame scale pass turns them into factors f_j
  const float* e_own;      // (B, T+1, C)
  const float* s_out;      // (B, T+1, C)
  const float* halo;       // (B*P, Kmax, C), or null when the scan took each end sum from the tables
  const double* db_part;   // (B*P, Kmax, C)
  double* tr_part;         // (B*GNB, C, C)
  // coverage pass: inputs, the forward's levels and log2 Z, the backward chunks'
  // recorded beta states (positions t_lo .. t_lo+Kmax-1 of chunk j >= 1)
  const float* cum;        // (B, T+1, C)
  const float* emit;       // (B, T, C) projected scores in place of cum, or null
  const float* db;         // (K, C)
  const float* ps;         // (B, T, C) or null
  const double* alvl;      // (B, T+1)
  const double* z2;        // (B)
  const float* st_end;     // (B*P, Kmax, C)
  const double* lv_end;    // (B*P, Kmax)
  const float* grad_output;
  float* grad_cum;
  float* grad_ps;
  float* grad_pe;
  float* grad_tr;
  float* grad_db;
  int shift;               // 1: grad_cum is (B, T, C) and row t >= 1 goes to row t-1 (row 0 is dropped)
  // bounded-memory backward: add the window's rows and shared gradients into the
  // outputs (accum); cum / ps and the row outputs point at the window's first
  // row of sequence 0, sequence b's rows xseq (cum, grad_cum) / pseq (ps and
  // the projection gradients) elements further (0: the window's own T).
  // Chunk 0 of a sequence with a handed-over start state (org_ok[b]) keeps its
  // frame factor (position 0 is not the sequence start), and so does a chunk
  // whose coverage segments may end beyond the window when the sequence goes
  // on (end_ok[b])
  int accum;
  const int* org_ok;
  const int* end_ok;
  int64_t xseq, pseq;
};

struct ViterbiParams {
  const float* cum;
  const float* trans;
  const float* db;
  const int64_t* lengths;
  const float* ps;
  const float* pe;
  int B, T, C, K, Kmax, RS;
  float* score;        // (B) Viterbi score (max over final labels)
  int32_t* bp;         // (B, T+1, C) packed backpointer (k << 16 | c_src), or null
  int32_t* final_c;    // (B) first argmax label at position len
  int trows;           // transition is (trows, C, C), indexed by duration, when > 0
};

// Gold-path score (segmentation implied by per-position labels) and its gradients.
struct GoldParams {
  const float* cum;        // (B, T+1, C)
  const float* emit;       // (B, T, C) projected scores in place of cum, or null
  int emit_grad;           // backward: gcum is the (B, T, C) gradient of the projected scores
  const float* tr;         // (C, C)
  const float* db;         // (Kdb, C)
  const int64_t* labels;   // (B, T)
  const int64_t* lengths;  // (B,)
  int B, T, C, K, Kdb;
  int NCH;                 // position blocks per sequence
  int H;                   // label lookback staged per block (set by the launcher)
  double* part;            // (B, NCH) block partial scores
  int* bad;                // (B, NCH) out-of-range label flags
  float* score;            // (B)
  // backward
  const float* gout;       // (B)
  float* gcum;             // (B, T+1, C)
  int* cnt;                // (B, NHIST) segment / transition counts
  int NHIST;               // Kdb*C + C*C
  float* gtr;              // (C, C)
  float* gdb;              // (Kdb, C)
};

// Emission prologue: projected scores -> cumulative scores (and backward).
struct PrologueParams {
  const void* x;     // (B, T, C) scores, dtype TSM_DTYPE_*
  int dtype;
  const float* g;    // backward: gradient of cum, row u of sequence b at g[(b*GR + u + goff)*C]
  int GR, goff;      // (T+1, 0) for a (B, T+1, C) tensor; (T, -1) for row u kept at u-1 of a (B, T, C) one
  float* cum;        // (B, T+1, C)
  float* gx;         // backward: (B, T, C)
  double* part;      // (B, NBL, C) block sums, then carries
  double* part2;     // (B, NBL, C) backward: position-weighted block sums
  double* mean;      // (B, C) centring term
  int B, T, C, NBL;
  int centre;
};

// launchers (return hipError_t as int)
int launch_scan_forward(const Plan& pl, const ScanParams& p, int semiring, hipStream_t s);
int launch_scan_backward(const Plan& pl, const ScanParams& p, int semiring, hipStream_t s);
// VGPRs of the register-resident scan kernel a launch with this plan would use
// (kind 0: log forward, 1: log backward with separate marginals, 2: Viterbi
// forward), -1 when unknown
int fast_scan_regs(const Plan& pl, int kind);
// backward log scan with fused marginals (pl.mfused), and its row passes
int launch_scan_backward_fused(const Plan& pl, const ScanParams& p, hipStream_t s);
int launch_fused_j16_lo(const Plan& pl, const ScanParams& p, hipStream_t s);
int launch_fused_j16_hi(const Plan& pl, const ScanParams& p, hipStream_t s);
int launch_u_rows(const Plan& pl, const FusedParams& f, hipStream_t s);
int launch_fused_finalize(const Plan& pl, const FusedParams& f, hipStream_t s);
// verification of speculative chunk boundaries / level offsets (shared by both scan paths)
// after_retry: the verification that follows the retry pass (nothing to do unless it reran a chunk)
int launch_verify(const Plan& pl, const ScanParams& p, bool forward, hipStream_t s, bool after_retry = false);
int launch_apply_offsets(const Plan& pl, const ScanParams& p, bool forward, hipStream_t s);
// register-resident log-semiring scan, one entry per lane-group size (pl.FJ)
int launch_fast_j8(const Plan& pl, const ScanParams& p, bool forward, hipStream_t s);
int launch_fast_j16(const Plan& pl, const ScanParams& p, bool forward, hipStream_t s);
int launch_fast_j16_lo(const Plan& pl, const ScanParams& p, bool forward, hipStream_t s);
int launch_fast_j16_hi(const Plan& pl, const ScanParams& p, bool forward, hipStream_t s);
int launch_fast_j32(const Plan& pl, const ScanParams& p, bool forward, hipStream_t s);
int launch_fast_j64(const Plan& pl, const ScanParams& p, bool forward, hipStream_t s);
// max-semiring forward with backpointers (factorised Viterbi), per lane-group size
int launch_fast_max_j8(const Plan& pl, const ScanParams& p, hipStream_t s);
int launch_fast_max_j16(const Plan& pl, const ScanParams& p, hipStream_t s);
int launch_fast_max_j16_lo(const Plan& pl, const ScanParams& p, hipStream_t s);
int launch_fast_max_j16_hi(const Plan& pl, const ScanParams& p, hipStream_t s);
int launch_fast_max_j32(const Plan& pl, const ScanParams& p, hipStream_t s);
int launch_fast_max_j64(const Plan& pl, const ScanParams& p, hipStream_t s);
// cooperative log-semiring scan (tsm_coop.hip), pl.CR durations per lane
int launch_coop_scan(const Plan& pl, const ScanParams& p, bool forward, bool logsr, hipStream_t s);
int launch_scan_viterbi(const Plan& pl, const ScanParams& p, hipStream_t s);
// Chunked speculative backtrace (tsm_backtrace.hip): P chunks of Lc positions per
// sequence, walks starting D positions above their chunk, TCH backpointer rows
// per LDS stage (0: rows read from global memory).
constexpr int kBtMaxChunks = 512;
struct BtPlan {
  int P, Lc, D, TCH;
};
BtPlan backtrace_plan(int B, int T, int C, int Kmax);
size_t backtrace_ws_bytes(const BtPlan& bp, int B);
// bp in the exact format (k << 16 | c_prev); the path starts at (len, first
// maximiser of fin[b, :]) when fin is given, else at (len, final_c[b])
int launch_backtrace(const BtPlan& bpl, const int32_t* bp, const float* fin, const int32_t* final_c,
                     const int64_t* lengths, int B, int T, int C, int Kmax, void* ws, int32_t* seg_count,
                     int32_t* segs, hipStream_t s);
// score terms of traceback rows: (B, T, 6) fp64 (start, end, label, content, duration bias, transition)
int launch_segment_terms(const float* cum, const float* tr, const float* db, const int32_t* seg_count,
                         const int32_t* segs, int B, int T, int C, int K, double* out, hipStream_t s);
// factorised backpointers (k* ending at t | c'* starting at t) to the exact format
int launch_fact_to_exact(const int32_t* bp, const int64_t* lengths, int B, int T, int C, int32_t* out,
                         hipStream_t s);
// register-resident marginals (16 lanes per label, pl.MR durations per lane)
int launch_margfast_j16(const Plan& pl, const MargParams& q, hipStream_t s);
int launch_margfast_j16_lo(const Plan& pl, const MargParams& q, hipStream_t s);
int launch_margfast_j16_hi(const Plan& pl, const MargParams& q, hipStream_t s);
int launch_margfast_j16_wide(const Plan& pl, const MargParams& q, hipStream_t s);  // 64 < C <= 128
int launch_marginals(const Plan& pl, const MargParams& q, hipStream_t s);
int launch_finalize(const Plan& pl, const FinalParams& f, hipStream_t s);
int launch_block_coverage(const Plan& pl, const MargParams& q, double* bscale, hipStream_t s);
int launch_viterbi(const Plan& pl, const ViterbiParams& v, hipStream_t s);
// duration-dependent transitions: log2-scaled tables of both directions
// (trf [k-1][c_dst][c_src], trb [k-1][c_src][c_dst]), dense scans and marginals
int launch_dense_prep(const Plan& pl, const float* trans, float* trf, float* trb, hipStream_t s);
int launch_dense_scan(const Plan& pl, const ScanParams& p, int semiring, bool forward, hipStream_t s);
int launch_dense_marginals(const Plan& pl, const MargParams& q, hipStream_t s);
int prologue_blocks(int T);
int launch_prologue(const PrologueParams& q, bool bwd, hipStream_t s);
int gold_chunks(int T);
size_t gold_lds_bytes(int K);
int launch_gold_score(const GoldParams& g, hipStream_t s);
int launch_gold_backward(const GoldParams& g, hipStream_t s);
int launch_checkpoints(const float* aval, const double* alvl, const int64_t* lengths, int B, int T,
                       int C, int K, int S, int n_ckpt, float* out, hipStream_t s);
// bounded-memory backward (tsm_window.hip)
int launch_window_setup(const int64_t* lengths, int B, int T, int Wlen, int nw, int64_t* lenw, int* okf, int* okb,
                        hipStream_t s);
int launch_ck_extract(const float* st_end, const double* lv_end, const double* offs, int B, int P, int Wc, int Kmax,
                      int C, int nw, float* ck_st, double* ck_lv, double* ck_al, hipStream_t s);
int launch_window_row0(const float* ck_ah, const double* ck_al, const int* okf, int B, int Tw, int C, float* ah,
                       double* al, hipStream_t s);
int launch_window_state_fix(double* lv, const double* offs, int B, int P, int Kmax, hipStream_t s);
int launch_window_halo_add(const float* thalo, const float* halo, const double* mframe, const int64_t* lenw,
                           const int* okb, int B, int P, int Lc, int Kmax, int C, int rows, const float* gout,
                           float* gcum_e, float* gpe_e, int64_t xseq, int64_t pseq, hipStream_t s);
int launch_fill_zero(float* p, size_t n, hipStream_t s);

// Opt-in per-kernel timing.  Kernel ids index the totals of timing_read().
enum KernelId : int {
  kKScanFwd = 0,
  kKScanBwd,
  kKVerify,
  kKFwdFixup,
  kKBwdFixup,
  kKApplyOffsets,
  kKMarginal,
  kKFinalizeRows,
  kKFinalizeShared,
  kKCheckpoints,
  kKViterbi,
  kKBacktrace,
  kKRetry,
  kKTransPrep,
  kKGold,
  kKPrologue,
  kKURows,
  kKTransGrad,
  kKFusedRows,
  kKFusedShared,
  kKCoverage,
  kNumKernels
};

// Brackets the launches made during its lifetime with events on stream `s`
// (a no-op unless timing is enabled).
class TimedLaunch {
 public:
  TimedLaunch(int id, hipStream_t s);
  ~TimedLaunch();
  TimedLaunch(const TimedLaunch&) = delete;
  TimedLaunch& operator=(const TimedLaunch&) = delete;

 private:
  int id_;
  hipStream_t s_;
  hipEvent_t a_, b_;
};

int timing_enable(int on);
int timing_read(double* total_ms, int64_t* launches, int n);
const char* timing_name(int id);

}  // namespace tsm
