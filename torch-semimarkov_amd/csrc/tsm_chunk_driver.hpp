// Driver of a chunked, speculative scan direction, shared by every scan whose
// chunk body follows the same contract (the register-resident log scan and
// the dense scan of duration-dependent transitions).
//
// A chunk type CH provides
//   static constexpr bool kFwd;          // direction
//   static constexpr bool kLog;          // log semiring (else max)
//   static constexpr int kMaxThreads;    // launch bound of its kernels
//   __device__ static void run(const ScanParams&, char* smem, int b, int j, int mode,
//                              const float* init_st, const double* init_lv);
//   __device__ static double* red(char* smem, const ScanParams&);  // >= 64 doubles of LDS
// where run() computes chunk j of sequence b in mode 0 (exact from the
// sequence start / end), 1 (speculative from a flat state W positions early)
// or 2 (exact from the boundary state (init_st, init_lv)), records boundary
// states for verification and writes the chunk's outputs in its own frame.
//
// One direction is: the parallel pass over all chunks, the verification of
// every speculative boundary together with a parallel retry (4x warm-up) of the
// chunks that fail it, verification again when something reran, a sequential
// per-sequence repair (exact recompute of what still fails, accumulation of
// frame offsets), and the application of the offsets to the stored levels.
#pragma once

#include "tsm_scan_common.hpp"

namespace tsm {
namespace scan_detail {

// Parallel pass of one direction: one block per chunk, exact or speculative.
template <class CH>
__device__ __forceinline__ void chunk_scan_body(const ScanParams& p) {
  extern __shared__ __align__(16) char smem[];
  constexpr bool FWD = CH::kFwd;
  const int b = blockIdx.x / p.P, j = blockIdx.x % p.P;
  const int len = seq_len(p, b);
  const int item = b * p.P + j;
  if (FWD ? (j > 0 && j * p.Lc >= len) : (j > bwd_last_chunk(p, len))) {
    if (threadIdx.x == 0) p.status[item] = -1;  // empty chunk
    return;
  }
  if (p.retry) {
    // verification of a speculative chunk against its neighbour's end state (the
    // (max, min) spread, kept for the repair); rerun with the longer warm-up when it
    // fails.  A neighbour that reruns here rewrites that end state meanwhile: a spread
    // measured from a half-rewritten state is measured again by the second
    // verification, which runs because the neighbour reran, before the repair uses it.
    if (p.status[item] != 1) return;
    const size_t e = FWD ? (size_t)(item - 1) : (size_t)(item + 1);
    double hi, lo, dmax, dmin;
    boundary_spread_part(p, e, (size_t)item, hi, lo);
    block_minmax(hi, lo, CH::red(smem, p), dmax, dmin);
    if (threadIdx.x == 0) {
      p.vstat[2 * item] = dmax;
      p.vstat[2 * item + 1] = dmin;
    }
    if (dmax - dmin <= (double)p.tol) return;
  } else if (blockIdx.x == 0 && threadIdx.x == 0) {
    *p.vflag = 0;  // the retry pass sets it when it reruns a chunk
  }
  const int mode = (FWD ? fwd_spec(p, j) : bwd_spec(p, j, len)) ? 1 : 0;
  if (threadIdx.x == 0) {
    p.status[item] = mode;
    if (p.retry) *p.vflag = 1;
  }
  CH::run(p, smem, b, j, mode, nullptr, nullptr);
}

template <class CH>
__global__ void __launch_bounds__(CH::kMaxThreads) chunk_scan_kernel(ScanParams p) {
  chunk_scan_body<CH>(p);
}

// The retry pass (p.retry = 1): the same body under its own name, so that
// profilers report the main pass and the retry separately.
template <class CH>
__global__ void __launch_bounds__(CH::kMaxThreads) chunk_retry_kernel(ScanParams p) {
  chunk_scan_body<CH>(p);
}

// Fast path of the repair: when no speculative chunk of sequence b failed its
// verification, nothing is recomputed and the frame offsets are a segmented
// prefix sum over the walk (restarting at 0 at each exact chunk) of the
// accepted mid-spreads.  Wave 0 scans 64 chunks at a time with shuffles.
// Returns false (and writes nothing) when some chunk needs a recompute;
// otherwise F (thread 0) is the offset after the walk.
template <bool FWD>
__device__ bool fixup_prefix(const ScanParams& p, int b, int jl, int nch, double& F) {
  const int n = FWD ? nch - 1 : jl;  // chunks of the walk: FWD 1..nch-1, BWD jl-1..0
  bool bad = false;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    const int it = b * p.P + (FWD ? 1 + i : jl - 1 - i);
    bad = bad || (p.status[it] == 1 && !(p.vstat[2 * it] - p.vstat[2 * it + 1] <= (double)p.tol));
  }
  if (__syncthreads_or(bad)) return false;
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    double carry = 0.0;
    for (int i0 = 0; i0 < n; i0 += 64) {
      const int i = i0 + lane;
      const int it = b * p.P + (FWD ? 1 + i : jl - 1 - i);
      double v = 0.0;
      int rst = 0;
      if (i < n) {
        if (p.status[it] == 1) v = 0.5 * (p.vstat[2 * it] + p.vstat[2 * it + 1]);
        else rst = 1;  // exact chunk: the offset restarts at 0
      }
      // inclusive segmented scan: (a, ra) then (v, r) -> (r ? v : a + v, ra | r)
      for (int d = 1; d < 64; d <<= 1) {
        const double a = __shfl_up(v, d, 64);
        const int ra = __shfl_up(rst, d, 64);
        if (lane >= d) {
          if (!rst) v += a;
          rst |= ra;
        }
      }
      const double off = rst ? v : carry + v;
      if (i < n) p.offs[it] = off;
      carry = __shfl(off, 63, 64);
    }
    F = carry;
  }
  return true;
}

// Sequential verification / repair of one direction: one block per sequence
// walks its chunks, accepts a speculative chunk's frame offset when the
// boundary spread is within tolerance, recomputes it exactly otherwise.
template <class CH>
__global__ void __launch_bounds__(CH::kMaxThreads) chunk_fixup_kernel(ScanParams p) {
  extern __shared__ __align__(16) char smem[];
  constexpr bool FWD = CH::kFwd;
  const int b = blockIdx.x;
  const int len = seq_len(p, b);
  double* red = CH::red(smem, p);
  const int Kmax = p.Kmax, C = p.C;
  double F = 0.0;
  int n_re = 0;
  bool prev_recomputed = false;
  const int jl = bwd_last_chunk(p, len);
  const int nch = len == 0 ? 1 : (len + p.Lc - 1) / p.Lc;
  if (threadIdx.x == 0) p.offs[(size_t)b * p.P + (FWD ? 0 : jl)] = 0.0;
  if (fixup_prefix<FWD>(p, b, jl, nch, F)) {
    __syncthreads();
    if (FWD) finish_partition<CH::kLog>(p, b, len, F, 0);
    else if (threadIdx.x == 0 && p.recomputed != nullptr) p.recomputed[b] = 0;
    return;
  }
  for (int j = FWD ? 1 : jl - 1; FWD ? j < nch : j >= 0; j += FWD ? 1 : -1) {
    const int item = b * p.P + j;
    if (p.status[item] != 1) {
      F = 0.0;  // the chunk ran exactly from the sequence end
      prev_recomputed = false;
    } else {
      const size_t e = FWD ? (size_t)(item - 1) : (size_t)(item + 1), sp = (size_t)item;
      double dmax, dmin;
      if (!prev_recomputed) {
        // measured in parallel by verify_kernel against the neighbour's original end state
        dmax = p.vstat[2 * sp];
        dmin = p.vstat[2 * sp + 1];
      } else {
        // the neighbour was recomputed here: its end state changed, measure again
        double hi, lo;
        boundary_spread_part(p, e, sp, hi, lo);
        block_minmax(hi, lo, red, dmax, dmin);
      }
      if (dmax - dmin <= (double)p.tol) {
        F += 0.5 * (dmax + dmin);
        prev_recomputed = false;
      } else {
        CH::run(p, smem, b, j, 2, p.st_end + e * Kmax * C, p.lv_end + e * Kmax);
        __syncthreads();
        ++n_re;
        prev_recomputed = true;
        if (threadIdx.x == 0) p.status[item] = 2;
      }
    }
    if (threadIdx.x == 0) p.offs[(size_t)item] = F;
  }
  __syncthreads();
  if (FWD) {
    finish_partition<CH::kLog>(p, b, len, F, n_re);
  } else if (threadIdx.x == 0 && p.recomputed != nullptr) {
    p.recomputed[b] = n_re;
  }
}

// Launch of one direction: parallel pass, verification, retry, sequential
// repair, level offsets.  `lds` bytes of dynamic LDS and `nthreads` threads
// (<= CH::kMaxThreads) per block.
template <class CH>
int launch_chunk_dir(const Plan& pl, const ScanParams& p, size_t lds, int nthreads, hipStream_t st) {
  constexpr bool fwd = CH::kFwd;
  auto k = chunk_scan_kernel<CH>;
  auto kr = chunk_retry_kernel<CH>;
  auto kf = chunk_fixup_kernel<CH>;
  if (p.query_regs != nullptr) {
    hipFuncAttributes a;
    const hipError_t qe = hipFuncGetAttributes(&a, (const void*)k);
    *p.query_regs = qe == hipSuccess ? a.numRegs : -1;
    (void)hipGetLastError();
    return hipSuccess;
  }
  hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  e = hipFuncSetAttribute((const void*)kr, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  e = hipFuncSetAttribute((const void*)kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  {
    TimedLaunch tl(fwd ? kKScanFwd : kKScanBwd, st);
    hipLaunchKernelGGL(k, dim3(pl.B * pl.P), dim3(nthreads), lds, st, p);
  }
  if (pl.P > 1) {
    // verification of every speculative chunk, and those that fail again, in
    // parallel, with a longer warm-up
    {
      TimedLaunch tl(kKRetry, st);
      hipLaunchKernelGGL(kr, dim3(pl.B * pl.P), dim3(nthreads), lds, st, retry_params(p));
    }
    e = (hipError_t)launch_verify(pl, p, fwd, st, true);
    if (e != hipSuccess) return e;
  }
  {
    TimedLaunch tl(fwd ? kKFwdFixup : kKBwdFixup, st);
    hipLaunchKernelGGL(kf, dim3(pl.B), dim3(nthreads), lds, st, p);
  }
  e = (hipError_t)launch_apply_offsets(pl, p, fwd, st);
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

}  // namespace scan_detail
}  // namespace tsm
