/*
 * tsm_hip.h -- C ABI of libtsm_hip.so, the MI355X (gfx950) streaming
 * semi-Markov CRF scan.
 *
 * All pointers are device pointers (HIP) unless stated otherwise; all arrays
 * are dense row-major fp32 / int64 / fp64 as documented.  No entry point
 * allocates memory: callers pass a workspace of at least the size reported by
 * the matching *_workspace() query.  Work is enqueued on `stream` (a
 * hipStream_t, may be NULL for the default stream) and is asynchronous.
 * Every function returns 0 on success or a TSM_ERR_* code; the message of the
 * last failure on the calling thread is available from tsm_last_error().
 *
 * Conventions (reference: biobenkj/torch-semimarkov README.md:96-125,
 * src/torch_semimarkov/streaming/pytorch_reference.py:86-111):
 *   cum_scores      (B, T+1, C)  cumulative projected scores, row 0 = 0
 *   transition      (C, C)       transition[c_src][c_dst], or with trans_rows > 0
 *                   (trans_rows, C, C)  transition[k][c_src][c_dst] for a segment of
 *                                duration k (reference pytorch_reference.py:104-109,
 *                                triton_forward.py:613-616 has_duration_transitions);
 *                                durations 1..max(K-1,1) are used, so trans_rows
 *                                must be >= max(K-1,1)+1; C <= 128
 *   duration_bias   (K, C)       K = max_duration; durations 1..K-1 use row
 *                                min(k, K-1); K = 1 uses duration 1, row 0
 *   lengths         (B,) int64   0 <= lengths[b] <= T (clamped on device)
 *   proj_start/end  (B, T, C) or NULL   boundary scores at segment start / end
 *   semiring        TSM_SEMIRING_LOG (logsumexp) or TSM_SEMIRING_MAX
 */
#ifndef TSM_HIP_H
#define TSM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TSM_OK 0
#define TSM_ERR_INVALID 1     /* bad argument (shape, size, null pointer) */
#define TSM_ERR_UNSUPPORTED 2 /* valid but not implemented on this path */
#define TSM_ERR_HIP 3         /* HIP runtime error */
#define TSM_ERR_WORKSPACE 4   /* workspace smaller than required */

#define TSM_SEMIRING_LOG 0
#define TSM_SEMIRING_MAX 1

#define TSM_DTYPE_F32 0
#define TSM_DTYPE_BF16 1
#define TSM_DTYPE_F16 2

#define TSM_VITERBI_AUTO 0       /* factorised for large or long problems when it fits, else exact */
#define TSM_VITERBI_EXACT 1      /* the reference's fp32 operation order, bit-identical scores */
#define TSM_VITERBI_FACTORISED 2 /* K*C + C^2 terms per step, chunked over all CUs */

/* Library version (major*10000 + minor*100 + patch). */
int tsm_version(void);

/* Message of the last error on the calling thread ("" if none).  Host pointer. */
const char* tsm_last_error(void);

/*
 * Launch plan for a problem shape, for diagnostics and tests.  Fills up to
 * `n` int64 host values: J, NT, RS, P, Lc, W, global_rings, scan_lds, NB, TB,
 * CB, NCB, JM, NTM, marg_lds, Kmax, n_cu, R, KP, RMAX, fast, FJ, FR, FNT,
 * fast_lds, mfast, MR, dense, DJ, DNT, dtrl, dense_lds, DG, DNTM, DNB, DTB,
 * dmarg_lds, coop, CG, CCL, CR, CNQ, coop_lds, mfused, GNB, GTB, P2, Lc2, FRL2, fast_lds2,
 * dualF, dualB, dualV, regsF, regsB, regsV (fast = 1: log-semiring scans use
 * the register-resident kernels with
 * FJ lanes per label and FR durations per lane; mfast = 1: the marginals use
 * the register-resident kernel with MR durations per lane; the environment
 * variable TSM_SCAN_PATH=generic turns both off; dense = 1: duration-dependent
 * transitions, dense scans with DJ lanes per label, transitions in LDS when
 * dtrl = 1, dense marginals in DNB blocks of DTB positions; coop = 1: rings too
 * large for one CU, log-semiring scans run on groups of CG cooperating blocks
 * with CCL labels each and CR durations per lane, CNQ co-resident groups;
 * mfused = 1: the log-semiring backward computes the segment marginals inside
 * the register-resident beta scan, transition gradient in GNB row blocks of GTB
 * starts per sequence; TSM_MARGINAL_PATH=separate turns it off; dualF / dualB /
 * dualV = 1: the log forward / the log backward with separate marginals / the
 * factorised Viterbi forward run two chunks per CU, P2 chunks of Lc2 positions
 * with rings of FRL2 entries (fast_lds2 bytes), because their kernels use
 * regsF / regsB / regsV VGPRs, few enough for two workgroups per CU; -1 = not
 * queried).
 */
int tsm_plan_info(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int has_proj_start,
                  int has_proj_end, int64_t* out, int n);

/* ---------------------------------------------------------------------------
 * Forward: log partition (semiring LOG) or Viterbi score of the factorised,
 * normalised recursion (semiring MAX), per sequence.
 * Replaces the reference's forward launchers:
 *   streaming/triton_forward.py:554-714  launch_streaming_triton_kernel
 *   streaming/pytorch_reference.py:116-273 semi_crf_streaming_forward_pytorch
 * Outputs:
 *   partition       (B,)        fp32, natural log units
 *   log2_partition  (B,)        fp64, base-2 units (NULL allowed); the backward needs it
 *   alpha_hat       (B, T+1, C) fp32 normalised alpha (base 2) or NULL
 *   alpha_level     (B, T+1)    fp64 per-position level (base 2) or NULL
 *   alpha = (alpha_hat + alpha_level) * ln 2.  Pass both non-NULL to keep the
 *   state a later tsm_backward() call needs; pass both NULL for inference.
 *   recomputed      (B,) int32  chunks recomputed by the verifier, or NULL; -1 marks a
 *                               sequence whose cooperative scan (label sets too large for
 *                               one CU) gave up its bounded wait for a partner block: its
 *                               results are NaN (the call still returns TSM_OK, the kernels
 *                               having exited normally)
 * ------------------------------------------------------------------------- */
int tsm_forward_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int semiring,
                          int has_proj_start, int has_proj_end, size_t* bytes);
int tsm_forward(const float* cum_scores, const float* transition, const float* duration_bias,
                const int64_t* lengths, const float* proj_start, const float* proj_end, int64_t B, int64_t T,
                int64_t C, int64_t K, int64_t trans_rows, int semiring, float* partition, double* log2_partition,
                float* alpha_hat, double* alpha_level, int32_t* recomputed, void* workspace,
                size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * tsm_forward without a workspace argument: for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference, whose launchers
 * always allocate through torch.
 * Same arguments, outputs and results as tsm_forward (the same kernels run);
 * the workspace is a static device array of TSM_NOALLOC_SCRATCH_BYTES in the
 * library, one per GPU, allocated when the library's code is loaded on that
 * GPU and held until the process ends.  The call allocates nothing (no
 * hipMalloc / hipFree, no allocating library routine).
 *   - A problem whose workspace (tsm_forward_workspace) exceeds
 *     TSM_NOALLOC_SCRATCH_BYTES is refused with TSM_ERR_UNSUPPORTED before
 *     anything is launched.
 *   - Every call on one GPU shares that GPU's scratch: calls that overlap in
 *     time on one GPU (different streams or threads without ordering) race and
 *     give wrong results.  Calls ordered on one stream are safe; each call
 *     initialises what it reads of the scratch.
 * ------------------------------------------------------------------------- */
#define TSM_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)
int tsm_forward_noalloc(const float* cum_scores, const float* transition, const float* duration_bias,
                        const int64_t* lengths, const float* proj_start, const float* proj_end, int64_t B,
                        int64_t T, int64_t C, int64_t K, int64_t trans_rows, int semiring, float* partition,
                        double* log2_partition, float* alpha_hat, double* alpha_level, int32_t* recomputed,
                        void* stream);

/* ---------------------------------------------------------------------------
 * Backward: gradients of sum_b grad_output[b] * partition[b].
 * Replaces:
 *   streaming/triton_backward.py:556-790  launch_streaming_triton_backward
 *   streaming/pytorch_reference.py:276-525 semi_crf_streaming_backward_pytorch
 *   streaming/autograd.py:134-150          grad_output scaling / einsum reduction
 * Inputs alpha_hat / alpha_level / log2_partition come from tsm_forward with
 * the same semiring (MAX gives the reference's "soft max-marginals").
 * Outputs (all fully written):
 *   grad_cum        (B, T+1, C)  already scaled by grad_output[b]
 *   grad_transition (C, C)       sum_b grad_output[b] * d/dtransition
 *                   (trans_rows, C, C) with duration-dependent transitions (matrices
 *                                that no duration uses get zeros)
 *   grad_duration_bias (K, C)
 *   grad_proj_start, grad_proj_end (B, T, C) or NULL
 * ------------------------------------------------------------------------- */
int tsm_backward_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int has_proj_start,
                           int has_proj_end, size_t* bytes);
int tsm_backward(const float* cum_scores, const float* transition, const float* duration_bias,
                 const int64_t* lengths, const float* proj_start, const float* proj_end, int64_t B, int64_t T,
                 int64_t C, int64_t K, int64_t trans_rows, int semiring, const float* alpha_hat,
                 const double* alpha_level,
                 const double* log2_partition, const float* grad_output, float* grad_cum,
                 float* grad_transition, float* grad_duration_bias, float* grad_proj_start,
                 float* grad_proj_end, int32_t* recomputed, void* workspace, size_t workspace_bytes,
                 void* stream);

/* ---------------------------------------------------------------------------
 * Viterbi: max-semiring score, optionally with an on-device backtrace.
 * Replaces:
 *   streaming/pytorch_reference.py:116-273 (semiring="max") -> score
 *   nn.py:444-531 SemiMarkovCRFHead._traceback_single        -> segments
 * algorithm:
 *   TSM_VITERBI_EXACT       the reference's fp32 operation order: scores are
 *                           bit-identical, one workgroup per sequence, K*C^2
 *                           terms per step;
 *   TSM_VITERBI_FACTORISED  max-plus factorisation over source labels, chunked
 *                           with verification like the log-semiring scan:
 *                           scores within 1e-5 relative, segmentations identical
 *                           when no two candidates tie;
 *   TSM_VITERBI_AUTO        factorised when the register-resident scan or the
 *                           cooperative scan (C <= 128, K <= 513; tsm_plan_info
 *                           coop = 1) fits and the problem has >= 2^28 cells
 *                           (B*T*K*C^2) or its plan cuts each sequence into
 *                           several chunks (tsm_plan_info P >= 2); exact
 *                           otherwise.  The exact kernel holds one sequence's
 *                           ring in LDS: C = 128 with K = 500 only runs
 *                           factorised.
 * Duration-dependent transitions (trans_rows > 0) always run the exact kernel
 * (the factorisation does not hold; TSM_VITERBI_FACTORISED is refused).
 * Ties: the smallest duration, then the first source label, then the first
 * final label (nn.py:472-501).
 * Outputs:
 *   score      (B,) fp32  max over final labels of alpha[len]
 *   seg_count  (B,) int32 number of segments (with_traceback only)
 *   segments   (B, T, 4) int32 rows (start, end inclusive, label, previous
 *              label), last segment first (with_traceback only)
 * ------------------------------------------------------------------------- */
int tsm_viterbi_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int with_traceback,
                          size_t* bytes);
int tsm_viterbi(const float* cum_scores, const float* transition, const float* duration_bias,
                const int64_t* lengths, const float* proj_start, const float* proj_end, int64_t B, int64_t T,
                int64_t C, int64_t K, int64_t trans_rows, float* score, int with_traceback, int algorithm,
                int32_t* seg_count,
                int32_t* segments, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Segment score terms of a traceback: row i < seg_count[b] of tsm_viterbi's
 * segments becomes out[b, i, :] = (start, end, label, content, duration bias,
 * transition), fp64:
 *   content    = cum_scores[b, end+1, label] - cum_scores[b, start, label]
 *                (the fp32 difference)
 *   duration   = duration_bias[min(end - start + 1, K - 1), label]
 *   transition = transition[previous label, label]  (static (C, C) transitions;
 *                the first segment's previous label is the best start label)
 * A segment's score is (content + duration) + transition in fp64.  Rows from
 * seg_count[b] on are not written.  No workspace.
 * Replaces:
 *   nn.py:532-555  SemiMarkovCRFHead._compute_segment_score (three .item()
 *                  reads per segment)
 * ------------------------------------------------------------------------- */
int tsm_segment_terms(const float* cum_scores, const float* transition, const float* duration_bias,
                      const int32_t* seg_count, const int32_t* segments, int64_t B, int64_t T, int64_t C,
                      int64_t K, double* out, void* stream);

/* ---------------------------------------------------------------------------
 * Emission prologue: projected scores (B, T, C) -> cumulative scores
 * (B, T+1, C) fp32 with a zero first row, optionally zero-centred per (b, c)
 * over all T positions, and its backward.
 * Replaces:
 *   nn.py:196-209  torch.zeros(B, T+1, C) + cumsum(scores.float(), dim=1)
 *   streaming/autograd.py:300-340, streaming/__init__.py:85-121  the
 *                  zero-centring recipe projected - projected.mean(dim=1)
 * scores may be fp32, bf16 or fp16 (dtype TSM_DTYPE_*); prefix sums are carried
 * in fp64 and rounded once to fp32.
 *   tsm_cum_scores_backward: grad_scores[b,t,c] = sum_{u>t} grad_cum[b,u,c]
 *   (minus its mean over t when centred), fp32.
 * One workspace size serves both calls.
 * ------------------------------------------------------------------------- */
int tsm_prologue_workspace(int64_t B, int64_t T, int64_t C, size_t* bytes);
int tsm_cum_scores(const void* scores, int dtype, int64_t B, int64_t T, int64_t C, int centre, float* cum_scores,
                   void* workspace, size_t workspace_bytes, void* stream);
int tsm_cum_scores_backward(const float* grad_cum, int64_t B, int64_t T, int64_t C, int centre, float* grad_scores,
                            void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Gold-path score: the score of the segmentation implied by per-position
 * labels (the other half of the head's loss), and its gradients.
 * Replaces:
 *   helpers.py:365-544  score_gold_vectorized (a Python batch loop with .item()
 *                       synchronisations, then gathers) and the autograd
 *                       backward of its gathers
 * Segments are the maximal runs of equal labels inside [0, len); a segment
 * [s, e] with label c scores cum[e+1,c] - cum[s,c] + duration_bias[clamp(e-s+1,
 * 1, K-1), c] + transition[c_prev, c] (no transition for the first segment;
 * K = 1 uses row 0; T = 1 uses row 1 when db_rows > 1, as the reference).
 *   labels          (B, T) int64, read inside [0, len) only
 *   duration_bias   (db_rows, C), db_rows >= K
 *   score           (B,) fp32, summed in fp64; NaN for a sequence holding a
 *                   label outside [0, C)
 *   grad_cum        (B, T+1, C) = grad_output[b] * (+1 at e+1 / -1 at s of each segment)
 *   grad_transition (C, C), grad_duration_bias (db_rows, C): counts weighted
 *                   by grad_output, summed over the batch
 * One workspace size serves both calls.
 * ------------------------------------------------------------------------- */
int tsm_gold_score_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t db_rows, size_t* bytes);
int tsm_gold_score(const float* cum_scores, const float* transition, const float* duration_bias,
                   const int64_t* labels, const int64_t* lengths, int64_t B, int64_t T, int64_t C, int64_t K,
                   int64_t db_rows, float* score, void* workspace, size_t workspace_bytes, void* stream);
int tsm_gold_score_backward(const int64_t* labels, const int64_t* lengths, int64_t B, int64_t T, int64_t C,
                            int64_t K, int64_t db_rows, const float* grad_output, float* grad_cum,
                            float* grad_transition, float* grad_duration_bias, void* workspace,
                            size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Emission input: forward, backward, Viterbi and gold-path score on the
 * projected scores (B, T, C) fp32, T >= 1, instead of cumulative scores.
 * Replaces the head's prologue + scan (nn.py:196-220: cum_scores built with
 * torch.zeros + cumsum, then semi_crf_streaming_forward) and its gold score
 * (nn.py:297, helpers.py:365-544) -- the emission prologue fused into the
 * scans' streamed loads (cum[t] = sum_{u<t} scores[u] in fp64, as the
 * prologue computes it).  Arguments and outputs as the cumulative-score entry
 * points, with:
 *   tsm_backward_emissions   grad_scores (B, T, C) = d/dscores, already scaled by
 *                            grad_output[b] (the suffix sums of the cum gradient)
 *   tsm_gold_score_emissions_backward  grad_scores[b,t,c] = grad_output[b] *
 *                            [t < len and labels[b,t] == c]
 * The register-resident scans and marginals read the scores themselves and
 * build no (B, T+1, C) tensor; plans that run other kernels (tsm_plan_info:
 * fast = 0, coop = 1 or dense = 1, the max semiring forward / backward, the
 * exact Viterbi kernel) build cum in the workspace first.  The gold score uses
 * the workspace of tsm_gold_score_workspace.
 * ------------------------------------------------------------------------- */
int tsm_forward_emissions_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int semiring,
                                    int has_proj_start, int has_proj_end, size_t* bytes);
int tsm_forward_emissions(const float* scores, const float* transition, const float* duration_bias,
                          const int64_t* lengths, const float* proj_start, const float* proj_end, int64_t B,
                          int64_t T, int64_t C, int64_t K, int64_t trans_rows, int semiring, float* partition,
                          double* log2_partition, float* alpha_hat, double* alpha_level, int32_t* recomputed,
                          void* workspace, size_t workspace_bytes, void* stream);
int tsm_backward_emissions_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows, int semiring,
                                     int has_proj_start, int has_proj_end, size_t* bytes);
int tsm_backward_emissions(const float* scores, const float* transition, const float* duration_bias,
                           const int64_t* lengths, const float* proj_start, const float* proj_end, int64_t B,
                           int64_t T, int64_t C, int64_t K, int64_t trans_rows, int semiring,
                           const float* alpha_hat, const double* alpha_level, const double* log2_partition,
                           const float* grad_output, float* grad_scores, float* grad_transition,
                           float* grad_duration_bias, float* grad_proj_start, float* grad_proj_end,
                           int32_t* recomputed, void* workspace, size_t workspace_bytes, void* stream);
int tsm_viterbi_emissions_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int64_t trans_rows,
                                    int with_traceback, int algorithm, size_t* bytes);
int tsm_viterbi_emissions(const float* scores, const float* transition, const float* duration_bias,
                          const int64_t* lengths, const float* proj_start, const float* proj_end, int64_t B,
                          int64_t T, int64_t C, int64_t K, int64_t trans_rows, float* score, int with_traceback,
                          int algorithm, int32_t* seg_count, int32_t* segments, void* workspace,
                          size_t workspace_bytes, void* stream);
int tsm_gold_score_emissions(const float* scores, const float* transition, const float* duration_bias,
                             const int64_t* labels, const int64_t* lengths, int64_t B, int64_t T, int64_t C,
                             int64_t K, int64_t db_rows, float* score, void* workspace, size_t workspace_bytes,
                             void* stream);
int tsm_gold_score_emissions_backward(const int64_t* labels, const int64_t* lengths, int64_t B, int64_t T,
                                      int64_t C, int64_t K, int64_t db_rows, const float* grad_output,
                                      float* grad_scores, float* grad_transition, float* grad_duration_bias,
                                      void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Bounded-memory (checkpointed) forward + backward, log semiring: the forward
 * keeps no alpha table, only per window start (windows of `window` positions,
 * whole chunks of the forward's plan) the scan's ring state there and the
 * alpha-hat row; the backward recomputes alpha one window at a time, top
 * window first, and runs the fused backward over that window from the state
 * the window above handed down.  Workspace: one window's tables instead of
 * O(B*T*C).  Replaces the memory scheme of
 *   streaming/pytorch_reference.py:380-423 (ring checkpoints every
 *   sqrt(T*K) positions, alpha recomputed per segment in the backward)
 * Static (C, C) transitions, cumulative-score input, plans with the 16-lane
 * register-resident scans and fused marginals (C <= 64, K <= 513); other
 * problems get TSM_ERR_UNSUPPORTED.
 *   tsm_checkpoint_plan   the longest window (a multiple of the chunk length)
 *                         whose backward workspace fits budget_bytes (0: about
 *                         eight windows; one chunk when nothing fits), the
 *                         window count nw = ceil(T / window), and the two
 *                         workspace sizes.  Every sequence's window w runs in
 *                         the same launches; the workspace grows with B.
 *   tsm_checkpointed_workspace  the two workspace sizes for a given window
 *   tsm_forward_checkpointed  partition / log2_partition as tsm_forward, and
 *                         ck_state (nw, B, Kmax, C) f32, ck_level (nw, B, Kmax)
 *                         f64, ck_alpha (nw, B, C) f32, ck_alpha_level (nw, B)
 *                         f64 (Kmax = max(K-1, 1); entries of window 0 unused)
 *   tsm_backward_checkpointed  the gradients of tsm_backward (same outputs,
 *                         fully written) from the inputs and the checkpoints
 * ------------------------------------------------------------------------- */
int tsm_checkpoint_plan(int64_t B, int64_t T, int64_t C, int64_t K, int has_proj_start, int has_proj_end,
                        size_t budget_bytes, int64_t* window, int64_t* n_windows, size_t* forward_workspace_bytes,
                        size_t* backward_workspace_bytes);
int tsm_checkpointed_workspace(int64_t B, int64_t T, int64_t C, int64_t K, int has_proj_start, int has_proj_end,
                               int64_t window, size_t* forward_workspace_bytes, size_t* backward_workspace_bytes);
int tsm_forward_checkpointed(const float* cum_scores, const float* transition, const float* duration_bias,
                             const int64_t* lengths, const float* proj_start, const float* proj_end, int64_t B,
                             int64_t T, int64_t C, int64_t K, int64_t window, float* partition,
                             double* log2_partition, float* ck_state, double* ck_level, float* ck_alpha,
                             double* ck_alpha_level, void* workspace, size_t workspace_bytes, void* stream);
int tsm_backward_checkpointed(const float* cum_scores, const float* transition, const float* duration_bias,
                              const int64_t* lengths, const float* proj_start, const float* proj_end, int64_t B,
                              int64_t T, int64_t C, int64_t K, int64_t window, const float* ck_state,
                              const double* ck_level, const float* ck_alpha, const double* ck_alpha_level,
                              const double* log2_partition, const float* grad_output, float* grad_cum,
                              float* grad_transition, float* grad_duration_bias, float* grad_proj_start,
                              float* grad_proj_end, void* workspace, size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------------------
 * Ring checkpoints in the reference's layout (B, n_ckpt, K, C), raw alpha in
 * natural log units, rebuilt from tsm_forward's alpha_hat/alpha_level.
 * Replaces the ring_checkpoints output of
 *   streaming/pytorch_reference.py:192-258 / triton_forward.py:643-648,711-712
 * ------------------------------------------------------------------------- */
int tsm_ring_checkpoints(const float* alpha_hat, const double* alpha_level, const int64_t* lengths, int64_t B,
                         int64_t T, int64_t C, int64_t K, int64_t checkpoint_interval, int64_t n_checkpoints,
                         float* out, void* stream);

/* ---------------------------------------------------------------------------
 * Opt-in kernel timing (benchmarks, diagnostics).  No counterpart in the
 * reference, which has no per-kernel timer; it exists so a benchmark can time
 * one kernel on the stream the library launches it on.
 *   tsm_timing_enable(1)  clears the totals and brackets every later kernel
 *                         launch with two hipEvents on its stream; (0) stops.
 *   tsm_timing_read       waits for the recorded events and fills, for kernel
 *                         ids 0..n-1, the total milliseconds and launch counts
 *                         (host arrays; either may be NULL).
 *   tsm_timing_kernel_count / tsm_timing_kernel_name  the kernel ids.
 * The timing state is process-wide (guarded by a mutex).
 * ------------------------------------------------------------------------- */
int tsm_timing_enable(int enable);
int tsm_timing_read(double* total_ms, int64_t* launches, int n);
int tsm_timing_kernel_count(void);
const char* tsm_timing_kernel_name(int kernel_id);

#ifdef __cplusplus
}
#endif

#endif /* TSM_HIP_H */
