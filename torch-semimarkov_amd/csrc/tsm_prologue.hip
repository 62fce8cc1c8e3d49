// Emission prologue: projected scores (B, T, C) -> cumulative scores
// (B, T+1, C) with a zero first row, optionally zero-centred per (b, c), and
// its backward, for gfx950.
//
// Reference: nn.py:196-209 (cum_scores[:, 1:] = cumsum(scores.float(), dim=1)
// into a zeroed (B, T+1, C) buffer) and the zero-centring its streaming API
// asks callers to apply first (streaming/autograd.py:300-340,
// streaming/__init__.py:85-121: projected - projected.mean(dim=1)).
//
//   forward : cum[b, 0, c] = 0,  cum[b, u, c] = sum_{t<u} (x[b,t,c] - centre * mean_t x[b,t,c])
//   backward: G[b,t,c] = sum_{u>t} g[b,u,c];  grad_x = G - centre * mean_t G
//             (g may also be held in grad_x itself, row u at row u-1: each thread
//             reads a row of its own column before it writes it, so that runs in place)
//             (sum_t G[t] = sum_u u * g[u], so the centring term is one more column sum)
//
// HBM-bound.  Three passes of reduce-then-scan: per block of TT positions
// (all labels of a row block) the column sums, then one thread per (b, c)
// scans the block sums in fp64, then every block rescans its tile with the
// carry and writes fp32 results.  Prefix sums are carried in fp64 and rounded
// once, so cum is the correctly rounded prefix sum of the fp32 inputs at any
// T (the reference's fp32 scan drifts with T).  Inputs may be fp32, bf16 or
// fp16 (the projection's output dtype); results are fp32.
//
// Thread mapping: a block owns TT positions x all C labels of one sequence; a
// thread owns label c = tid % CG and rows r = tid / CG, + RG, ... of the tile
// (CG = threads per row group, RG = NT / CG row groups): consecutive lanes read
// consecutive labels of one row, so loads and stores are coalesced along the
// row-major (t, c) layout.

#include <hip/hip_bf16.h>
#include <hip/hip_fp16.h>

#include "../../include/tsm_hip.h"
#include "tsm_device.hpp"
#include "tsm_internal.hpp"

namespace tsm {
namespace {

constexpr int kPNT = 256;  // threads per block
constexpr int kPTT = 256;  // positions per block

template <int DT>
__device__ __forceinline__ float load_x(const void* p, size_t i) {
  if constexpr (DT == TSM_DTYPE_F32) return static_cast<const float*>(p)[i];
  else if constexpr (DT == TSM_DTYPE_BF16) return __bfloat162float(static_cast<const __hip_bfloat16*>(p)[i]);
  else return __half2float(static_cast<const __half*>(p)[i]);
}

// Column sums of one tile: part[b][blk][c] = sum over the tile's rows of x (forward) or,
// backward, (sum of g, sum of u * g) over rows u of cum in the tile.
template <int DT, bool BWD>
__global__ void __launch_bounds__(kPNT) prologue_reduce_kernel(PrologueParams q) {
  __shared__ double red[kPNT];
  __shared__ double red2[kPNT];
  const int C = q.C, T = q.T, NBL = q.NBL;
  const int blk = blockIdx.x % NBL, b = blockIdx.x / NBL;
  const int cb = blockIdx.y;  // label block of up to kPNT labels
  const int c0 = cb * kPNT, nc = min(kPNT, C - c0);
  const int CG = nc, RG = kPNT / CG;
  const int tid = threadIdx.x;
  const int c = c0 + tid % CG, rg = tid / CG;
  const bool act = rg < RG;
  double s = 0.0, s2 = 0.0;
  // forward rows are positions t of x; backward rows are positions u = 1..T of g
  const int r0 = BWD ? 1 + blk * kPTT : blk * kPTT;
  const int r1 = BWD ? min(r0 + kPTT, T + 1) : min(r0 + kPTT, T);
  if (act) {
    for (int r = r0 + rg; r < r1; r += RG) {
      if constexpr (BWD) {
        const double v = (double)q.g[((size_t)b * q.GR + r + q.goff) * C + c];
        s += v;
        s2 += (double)r * v;
      } else {
        s += (double)load_x<DT>(q.x, ((size_t)b * T + r) * C + c);
      }
    }
  }
  red[tid] = s;
  red2[tid] = s2;
  __syncthreads();
  if (tid < CG) {
    double a = 0.0, a2 = 0.0;
    for (int i = 0; i < RG; ++i) {
      a += red[i * CG + tid];
      a2 += red2[i * CG + tid];
    }
    const size_t o = ((size_t)b * NBL + blk) * C + c0 + tid;
    q.part[o] = a;
    if (BWD) q.part2[o] = a2;
  }
}

// One thread per (b, c): exclusive prefix of the block sums (forward) or
// suffix (backward) in fp64, and the centring term.
template <bool BWD>
__global__ void prologue_carry_kernel(PrologueParams q) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= q.B * q.C) return;
  const int b = idx / q.C, c = idx % q.C;
  const int NBL = q.NBL, C = q.C;
  double run = 0.0, tot2 = 0.0;
  for (int i = 0; i < NBL; ++i) {
    const int blk = BWD ? NBL - 1 - i : i;
    const size_t o = ((size_t)b * NBL + blk) * C + c;
    const double v = q.part[o];
    q.part[o] = run;  // carry into this block
    run += v;
    if (BWD) tot2 += q.part2[o];
  }
  // forward: mean of x over T; backward: mean over t of G[t] = (sum_u u g[u]) / T
  q.mean[idx] = (BWD ? tot2 : run) / (double)q.T;
}

// Rescan of one tile with its carry.  Each thread scans its rows of one label
// sequentially in fp64 after the row groups' totals have been combined.
template <int DT, bool BWD>
__global__ void __launch_bounds__(kPNT) prologue_scan_kernel(PrologueParams q) {
  __shared__ double tot[kPNT];
  const int C = q.C, T = q.T, NBL = q.NBL;
  const int blk = blockIdx.x % NBL, b = blockIdx.x / NBL;
  const int cb = blockIdx.y;
  const int c0 = cb * kPNT, nc = min(kPNT, C - c0);
  const int CG = nc, RG = kPNT / CG;
  const int tid = threadIdx.x;
  const int c = c0 + tid % CG, rg = tid / CG;
  const bool act = rg < RG;
  // contiguous row range of this thread inside the tile
  const int rows = BWD ? min(kPTT, T + 1 - (1 + blk * kPTT)) : min(kPTT, T - blk * kPTT);
  const int per = (rows + RG - 1) / RG;
  const int ra = act ? min(rg * per, rows) : rows, rb = act ? min(ra + per, rows) : rows;
  const int base = BWD ? 1 + blk * kPTT : blk * kPTT;
  double s = 0.0;
  for (int i = ra; i < rb; ++i) {
    if constexpr (BWD) s += (double)q.g[((size_t)b * q.GR + base + i + q.goff) * C + c];
    else s += (double)load_x<DT>(q.x, ((size_t)b * T + base + i) * C + c);
  }
  tot[tid] = s;
  __syncthreads();
  if (!act) return;
  const size_t pc = ((size_t)b * NBL + blk) * C + c;
  const double mean = q.centre ? q.mean[(size_t)b * C + c] : 0.0;
  double carry = q.part[pc];
  if constexpr (!BWD) {
    for (int i = 0; i < rg; ++i) carry += tot[i * CG + tid % CG];
    if (blk == 0 && rg == 0) q.cum[(size_t)b * (T + 1) * C + c] = 0.0f;
    for (int i = ra; i < rb; ++i) {
      const int t = base + i;
      carry += (double)load_x<DT>(q.x, ((size_t)b * T + t) * C + c);
      q.cum[((size_t)b * (T + 1) + t + 1) * C + c] = (float)(carry - mean * (double)(t + 1));
    }
  } else {
    // suffix: rows after this thread's range come first
    for (int i = rg + 1; i < RG; ++i) carry += tot[i * CG + tid % CG];
    for (int i = rb - 1; i >= ra; --i) {
      const int u = base + i;  // grad_x[u-1] = sum of g over rows >= u
      carry += (double)q.g[((size_t)b * q.GR + u + q.goff) * C + c];
      q.gx[((size_t)b * T + u - 1) * C + c] = (float)(carry - mean);
    }
  }
}

template <int DT>
int launch_prologue_dt(const PrologueParams& q, bool bwd, hipStream_t s) {
  const dim3 grid(q.B * q.NBL, (q.C + kPNT - 1) / kPNT);
  TimedLaunch tl(kKPrologue, s);
  if (bwd) {
    hipLaunchKernelGGL((prologue_reduce_kernel<DT, true>), grid, dim3(kPNT), 0, s, q);
    hipLaunchKernelGGL(prologue_carry_kernel<true>, dim3((q.B * q.C + 255) / 256), dim3(256), 0, s, q);
    hipLaunchKernelGGL((prologue_scan_kernel<DT, true>), grid, dim3(kPNT), 0, s, q);
  } else {
    hipLaunchKernelGGL((prologue_reduce_kernel<DT, false>), grid, dim3(kPNT), 0, s, q);
    hipLaunchKernelGGL(prologue_carry_kernel<false>, dim3((q.B * q.C + 255) / 256), dim3(256), 0, s, q);
    hipLaunchKernelGGL((prologue_scan_kernel<DT, false>), grid, dim3(kPNT), 0, s, q);
  }
  return hipGetLastError();
}

}  // namespace

int prologue_blocks(int T) { return (T + kPTT - 1) / kPTT; }

int launch_prologue(const PrologueParams& q, bool bwd, hipStream_t s) {
  if (bwd) return launch_prologue_dt<TSM_DTYPE_F32>(q, true, s);
  switch (q.dtype) {
    case TSM_DTYPE_F32: return launch_prologue_dt<TSM_DTYPE_F32>(q, false, s);
    case TSM_DTYPE_BF16: return launch_prologue_dt<TSM_DTYPE_BF16>(q, false, s);
    case TSM_DTYPE_F16: return launch_prologue_dt<TSM_DTYPE_F16>(q, false, s);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace tsm
