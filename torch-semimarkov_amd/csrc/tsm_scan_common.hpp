// Chunk bookkeeping shared by the scan kernels (generic and register-resident):
// sequence lengths, which chunks run speculatively, the spread of a chunk
// boundary's (exact - speculative) state, and the partition from the final row.
#pragma once

#include "tsm_device.hpp"
#include "tsm_internal.hpp"

namespace tsm {
namespace scan_detail {

__device__ inline int seq_len(const ScanParams& p, int b) {
  int64_t L = p.lengths[b];
  if (L < 0) L = 0;
  if (L > p.T) L = p.T;
  return (int)L;
}

// Backward chunks own [j*Lc, (j+1)*Lc); the last one, jl, also owns position len.
// jl = (len-1)/Lc keeps jl < P even when len is a multiple of Lc.
__device__ inline int bwd_last_chunk(const ScanParams& p, int len) { return len > 0 ? (len - 1) / p.Lc : 0; }

// A forward chunk j >= 1 runs speculatively when its warm-up start t_lo - W has
// Kmax-1 real positions behind it; otherwise it runs exactly from position 0.
__device__ inline bool fwd_spec(const ScanParams& p, int j) { return j >= 1 && j * p.Lc - p.W >= p.Kmax - 1; }
// A backward chunk j < jl runs speculatively when its warm-up start t_hi + W
// has Kmax-1 real positions ahead of it; otherwise exactly from position len.
__device__ inline bool bwd_spec(const ScanParams& p, int j, int len) {
  const int jl = bwd_last_chunk(p, len);
  return j < jl && (j + 1) * p.Lc + p.W + p.Kmax - 1 <= len;
}


// Block-wide max / min of a double (all threads receive the result).
__device__ inline void block_minmax(double vmax, double vmin, double* red, double& omax, double& omin) {
  for (int m = 1; m < 64; m <<= 1) {
    vmax = fmax(vmax, __shfl_xor(vmax, m, 64));
    vmin = fmin(vmin, __shfl_xor(vmin, m, 64));
  }
  const int w = threadIdx.x >> 6, nw = (blockDim.x + 63) >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    red[w] = vmax;
    red[32 + w] = vmin;
  }
  __syncthreads();
  omax = red[0];
  omin = red[32];
  for (int i = 1; i < nw; ++i) {
    omax = fmax(omax, red[i]);
    omin = fmin(omin, red[32 + i]);
  }
  __syncthreads();
}

// Per-thread (max, min) of D[i,c] = (lv_end[e,i] - lv_spec[sp,i]) + (st_end[e,i,c] - st_spec[sp,i,c])
// over this thread's share of the Kmax*C boundary entries.  Entries unreachable
// in both states (< -1e8 in log2 units) are skipped: they add nothing to any sum.
__device__ inline void boundary_spread_part(const ScanParams& p, size_t e, size_t sp, double& hi, double& lo) {
  const int Kmax = p.Kmax, C = p.C, n = Kmax * C, nt = blockDim.x;
  hi = -1e300;
  lo = 1e300;
  auto take = [&](float a, float bb, double le, double ls) {
    if (a < -1e8f && bb < -1e8f) return;
    const double d = (le - ls) + ((double)a - (double)bb);
    hi = fmax(hi, d);
    lo = fmin(lo, d);
  };
  // four entries per thread loaded before any is used (the loads of one pass overlap)
  int idx = threadIdx.x;
  for (; idx + 3 * nt < n; idx += 4 * nt) {
    float a[4], bb[4];
    double le[4], ls[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int id = idx + u * nt, i = id / C;
      a[u] = p.st_end[e * n + id];
      bb[u] = p.st_spec[sp * n + id];
      le[u] = p.lv_end[e * Kmax + i];
      ls[u] = p.lv_spec[sp * Kmax + i];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) take(a[u], bb[u], le[u], ls[u]);
  }
  for (; idx < n; idx += nt) {
    const int i = idx / C;
    take(p.st_end[e * n + idx], p.st_spec[sp * n + idx], p.lv_end[e * Kmax + i], p.lv_spec[sp * Kmax + i]);
  }
}

// log2 partition of sequence b from the final row fin[b, :] (chunk-local frame
// fin_lvl[b] + F), written to z2 / zout by thread 0.  Threads 0..63 take part.
template <bool LOGSR>
__device__ inline void finish_partition(const ScanParams& p, int b, int len, double F, int n_re) {
  if (threadIdx.x >= 64) return;
  const int C = p.C;
  float m = kMinusInf;
  for (int cc = threadIdx.x; cc < C; cc += 64) m = fmax2(m, p.fin[(size_t)b * C + cc]);
  for (int k = 1; k < 64; k <<= 1) m = fmax2(m, __shfl_xor(m, k, 64));
  float r;
  if constexpr (LOGSR) {
    float sm = 0.0f;
    for (int cc = threadIdx.x; cc < C; cc += 64) sm += exp2_hw(p.fin[(size_t)b * C + cc] - m);
    for (int k = 1; k < 64; k <<= 1) sm += __shfl_xor(sm, k, 64);
    r = m + log2_hw(sm);
  } else {
    r = m;
  }
  if (threadIdx.x == 0) {
    if (p.recomputed != nullptr) p.recomputed[b] = n_re;
    if (len == 0) {
      // reference: the final alpha is never written -> reduction over NEG_INF
      p.z2[b] = (double)kNegInf * 1.4426950408889634;
      p.zout[b] = kNegInf;
    } else {
      const double z2 = p.fin_lvl[b] + F + (double)r;
      p.z2[b] = z2;
      p.zout[b] = (float)(z2 * kLn2);
    }
  }
}

// Parameters of the retry pass: failed speculative chunks run again with a 4x
// longer warm-up (exactly from the sequence end when that reaches it).
inline ScanParams retry_params(const ScanParams& p) {
  ScanParams q = p;
  q.retry = 1;
  q.W = 4 * p.W;
  return q;
}

}  // namespace scan_detail
}  // namespace tsm
