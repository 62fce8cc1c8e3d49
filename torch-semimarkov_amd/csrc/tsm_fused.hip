// Backward with the segment marginals fused into the register-resident beta
// scan (tsm_fastscan.hpp, MARG): the row passes around it.
//
//   u pass      u[t,c] = log2 sum_c' 2^(alpha-hat[t,c'] + trans[c',c] log2 e), the
//               forward side of a segment starting at t with label c (the scan
//               reads one value per step instead of redoing the label mix);
//   scan        per chunk j, in its own frame: end sums e_own (cumulative scores:
//               each owned row from the alpha table and the step's beta state;
//               emission input and windows: per-term sums, rows past the chunk
//               in halo), start sums
//               s_out, duration sums db_part, frame estimate mframe[j];
//   rows        grad_cum / grad_proj from E and S, each chunk's values times
//               f_j = 2^(mframe[j] + offs[j]) (offs: the chunk's verified
//               level offset), which takes them to probabilities;
//   transitions G[c',c] = sum_t 2^(alpha-hat[t,c'] + trans[c',c] log2 e - u[t,c]) S[t,c]
//               (the softmax weight of source c' times the start sum), per row
//               block in fp64;
//   coverage    every position lies in exactly one segment: the marginals of the
//               segments covering one position of each chunk sum to 1; the pass
//               measures that sum and divides the chunk's factor by it, which
//               removes the slowly varying scale error that rounding in the long
//               alpha / beta level chains leaves (see coverage_kernel);
//   shared      grad_db = sum_j f_j db_part[j], grad_tr = sum of the row blocks,
//               both weighted by grad_output, in a fixed order.
#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include "tsm_device.hpp"
#include "tsm_internal.hpp"

namespace tsm {
namespace {

constexpr double kLog2eD = 1.4426950408889634;

__device__ __forceinline__ int flen(const int64_t* lengths, int b, int T) {
  int64_t L = lengths[b];
  if (L < 0) L = 0;
  if (L > T) L = T;
  return (int)L;
}

// chunk owning row / start t of a sequence of length len (backward scan chunks)
__device__ __forceinline__ int fchunk(int t, int len, int Lc) {
  const int jl = len > 0 ? (len - 1) / Lc : 0;
  const int j = t / Lc;
  return j < jl ? j : jl;
}

// the chunk factor f_j (after the frame scale pass)
__device__ __forceinline__ double fscale(const FusedParams& f, int b, int j) { return f.mframe[(size_t)b * f.P + j]; }

// frame estimates -> factors f_j = 2^(fr_j + offs_j), in place
__global__ void frame_scale_kernel(FusedParams f) {
  const int n = f.B * f.P;
  for (int it = blockIdx.x * blockDim.x + threadIdx.x; it < n; it += gridDim.x * blockDim.x)
    f.mframe[it] = exp2(f.mframe[it] + f.offs[it]);
}

// ---- u pass: 64 rows per block, transitions and the rows' alpha-hat in LDS ----
// When every column's transition range is <= 30, u is a dot product:
// u[t,c] = cm[c] + log2 sum_c' 2^alpha-hat[t,c'] * 2^(tr[c',c] - cm[c]), both
// factors <= 1 and the largest term >= 2^-30 (alpha-hat has an exact 0 at the
// row's best label), so an underflowed 2^alpha-hat drops a term below 2^-96.
// A thread then keeps its column's factors in registers (CP >= C of them) and
// reads the rows' 2^alpha-hat as float4s: one FMA per pair, no exponential.
// Otherwise each pair takes an exponential (with a first pass for the row
// maximum when the range exceeds 64).
constexpr int kURows = 64;

template <int CP>
__global__ void __launch_bounds__(256) u_rows_kernel(FusedParams f) {
  extern __shared__ __align__(16) char smem[];
  const int C = f.C, T = f.T;
  const int b = blockIdx.y;
  const int len = flen(f.lengths, b, T);
  const int t0 = blockIdx.x * kURows;
  if (t0 > len) return;
  const int nr = min(kURows, len + 1 - t0);
  float* tr2 = reinterpret_cast<float*>(smem);  // [c_src][c_dst], log2 units
  float* ah = tr2 + C * C;                       // [row][c], row stride CP
  float* cmx = ah + kURows * CP;                 // [c] max over sources of tr2[., c]
  float* crg = cmx + C;                          // [c] its range (max - min)
  for (int i = threadIdx.x; i < C * C; i += blockDim.x) tr2[i] = f.trans[i] * kLog2e;
  __syncthreads();
  bool wide = false;
  for (int c = threadIdx.x; c < C; c += blockDim.x) {
    float hi = kMinusInf, lo = -kMinusInf;
    for (int cs = 0; cs < C; ++cs) {
      hi = fmax2(hi, tr2[cs * C + c]);
      lo = fmin(lo, tr2[cs * C + c]);
    }
    cmx[c] = hi;
    crg[c] = hi - lo;
    wide = wide || !(hi - lo <= 30.0f);
  }
  const bool fact = !__syncthreads_or(wide);
  const float* av = f.aval + ((size_t)b * (T + 1) + t0) * C;
  for (int i = threadIdx.x; i < nr * CP; i += blockDim.x) {
    const int r = i / CP, cs = i % CP;
    const float a = cs < C ? av[(size_t)r * C + cs] : kMinusInf;
    ah[i] = fact ? exp2_hw(a) : a;
  }
  __syncthreads();
  float* uo = f.uval + ((size_t)b * (T + 1) + t0) * C;
  if (fact) {
    const int RG = blockDim.x / C;  // row groups
    const int c = threadIdx.x % C, rg = threadIdx.x / C;
    if (rg >= RG) return;
    float er[CP];
#pragma unroll
    for (int cs = 0; cs < CP; ++cs) er[cs] = cs < C ? exp2_hw(tr2[cs * C + c] - cmx[c]) : 0.0f;
    for (int r = rg; r < nr; r += RG) {
      const float4* a4 = reinterpret_cast<const float4*>(ah + r * CP);
      float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
      for (int q = 0; q < CP / 4; ++q) {
        const float4 a = a4[q];
        s0 = fmaf(a.x, er[4 * q], s0);
        s1 = fmaf(a.y, er[4 * q + 1], s1);
        s0 = fmaf(a.z, er[4 * q + 2], s0);
        s1 = fmaf(a.w, er[4 * q + 3], s1);
      }
      uo[(size_t)r * C + c] = cmx[c] + log2_hw(s0 + s1);
    }
    return;
  }
  for (int i = threadIdx.x; i < nr * C; i += blockDim.x) {
    const int r = i / C, c = i % C;
    const float* a = ah + r * CP;
    const float* tc = tr2 + c;
    // Shift: alpha-hat <= 0 with an exact 0 at the row's best label, so every
    // term is <= 2^cmx[c] and the largest is >= 2^(cmx[c] - crg[c]): with a
    // range of at most 64 the column maximum is a safe shift (one pass);
    // otherwise the row's own maximum (a first pass).  Four independent chains
    // per pass (the LDS reads of a chain's next term overlap the others' work).
    int cs = 0;
    float m = cmx[c];
    if (!(crg[c] <= 64.0f)) {
      float m0 = kMinusInf, m1 = kMinusInf, m2 = kMinusInf, m3 = kMinusInf;
      for (; cs + 4 <= C; cs += 4) {
        m0 = fmax2(m0, a[cs] + tc[cs * C]);
        m1 = fmax2(m1, a[cs + 1] + tc[(cs + 1) * C]);
        m2 = fmax2(m2, a[cs + 2] + tc[(cs + 2) * C]);
        m3 = fmax2(m3, a[cs + 3] + tc[(cs + 3) * C]);
      }
      for (; cs < C; ++cs) m0 = fmax2(m0, a[cs] + tc[cs * C]);
      m = fmax2(fmax2(m0, m1), fmax2(m2, m3));
    }
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    for (cs = 0; cs + 4 <= C; cs += 4) {
      s0 += exp2_hw((a[cs] + tc[cs * C]) - m);
      s1 += exp2_hw((a[cs + 1] + tc[(cs + 1) * C]) - m);
      s2 += exp2_hw((a[cs + 2] + tc[(cs + 2) * C]) - m);
      s3 += exp2_hw((a[cs + 3] + tc[(cs + 3) * C]) - m);
    }
    for (; cs < C; ++cs) s0 += exp2_hw((a[cs] + tc[cs * C]) - m);
    uo[i] = m + log2_hw((s0 + s1) + (s2 + s3));
  }
}

// ---- coverage: every position lies in exactly one segment ----
// One block per backward chunk j >= 1 evaluates, at t_ref = t_lo - 1 (t_lo = j*Lc),
// cov_j = sum over the segments [s, s+k) covering t_ref (t_ref-Kmax < s <= t_ref < s+k,
// s+k <= len) and labels c of 2^(A[s,c] + seg(s,k,c) + beta_j[s+k,c] + offs_j - log2 Z)
// with A = alpha level + u (+ proj_start) and beta_j the chunk's own beta state at
// positions t_lo .. t_lo+Kmax-1, recorded for verification (st_end / lv_end).  In
// exact arithmetic cov_j = 1.  Rounding in the fp32 per-step results of the alpha /
// beta level chains (summed over up to 10^6 steps) leaves the marginals off by a
// slowly varying factor (measured up to ~5e-5 at T = 10^6); the chunk's marginals
// and this window share it, so the chunk factor f_j is divided by cov_j.  Chunk 0
// uses position 0, covered by the segments starting there (its start sums).  A
// value far from 1 (not a rounding drift) is left alone.
// LDS of coverage_kernel: ew (Kmax, C) fp32, the window's levels (Kmax) fp64, and,
// when they fit, the log2-scaled duration biases of durations 1..Kmax (Kmax, C).
inline size_t coverage_lds(int C, int Kmax, bool dbl) {
  return (size_t)Kmax * 8 + (size_t)Kmax * C * 4 * (dbl ? 2 : 1);
}

template <bool DBL>
__global__ void __launch_bounds__(1024) coverage_kernel(FusedParams f) {
  extern __shared__ __align__(16) char csm[];
  __shared__ double red[1024 / 64];
  const int b = blockIdx.y, j = blockIdx.x;
  const int C = f.C, T = f.T, Lc = f.Lc, K = f.K, Kmax = f.Kmax;
  const int len = flen(f.lengths, b, T);
  const int jl = len > 0 ? (len - 1) / Lc : 0;
  if (len == 0 || j > jl) return;
  double acc = 0.0;
  if (j == 0 && f.org_ok != nullptr && f.org_ok[b] != 0) {
    return;  // window of a longer sequence: position 0 is not covered by the starts there alone
  } else if (j >= 1 && f.end_ok != nullptr && f.end_ok[b] != 0 && j * Lc - 1 + Kmax > len) {
    return;  // window: segments covering t_ref may end in the window above
  } else if (j == 0) {
    for (int c = threadIdx.x; c < C; c += blockDim.x) acc += (double)f.s_out[(size_t)b * (T + 1) * C + c];
  } else {
    // lvs[i]: the chunk's level at t_lo + i; ew[i, c]: its beta state there plus the
    // content (cum[t_lo+i,c] - cum[t_ref,c]) log2 e (fp32: the level is kept apart);
    // dbl[k-1, c] = duration_bias[min(k, K-1), c] log2 e
    double* lvs = reinterpret_cast<double*>(csm);
    float* ew = reinterpret_cast<float*>(csm + (size_t)Kmax * 8);
    float* dbl = ew + (size_t)Kmax * C;
    const int t_lo = j * Lc, t_ref = t_lo - 1;
    const int s0 = max(0, t_ref - Kmax + 1);
    const size_t item = (size_t)b * f.P + j;
    const float* st = f.st_end + item * Kmax * C;
    const bool emit = f.emit != nullptr;
    const float* cum_b = emit ? nullptr : f.cum + (size_t)b * (f.xseq ? (size_t)f.xseq : (size_t)(T + 1) * C);
    const float* em_b = emit ? f.emit + (size_t)b * T * C : nullptr;
    const float* cref = emit ? nullptr : cum_b + (size_t)t_ref * C;
    const int ni = min(Kmax, len - t_lo + 1);  // positions t_lo .. min(len, t_lo+Kmax-1)
    for (int i = threadIdx.x; i < ni; i += blockDim.x) lvs[i] = f.lv_end[item * Kmax + i];
    if (emit) {
      // cum[t_lo+i] - cum[t_ref]: running sums of score rows t_ref .. t_lo+i-1, one thread per label
      for (int c = threadIdx.x; c < C; c += blockDim.x) {
        double run = 0.0;
        for (int i = 0; i < ni; ++i) {
          run += (double)em_b[(size_t)(t_ref + i) * C + c];
          ew[i * C + c] = st[i * C + c] + (float)(run * kLog2eD);
        }
      }
    } else {
      for (int idx = threadIdx.x; idx < ni * C; idx += blockDim.x) {
        const int i = idx / C, c = idx % C;
        ew[idx] = st[idx] + (cum_b[(size_t)(t_lo + i) * C + c] - cref[c]) * kLog2e;
      }
    }
    if constexpr (DBL) {
      for (int idx = threadIdx.x; idx < Kmax * C; idx += blockDim.x) {
        const int k = 1 + idx / C, c = idx % C;
        dbl[idx] = f.db[(size_t)(K == 1 ? 0 : min(k, K - 1)) * C + c] * kLog2e;
      }
    }
    __syncthreads();
    const double base = f.offs[item] - f.z2[b];
    const int n = (t_ref - s0 + 1) * C;
    for (int w = threadIdx.x; w < n; w += blockDim.x) {
      const int s = s0 + w / C, c = w % C;
      const double al = f.alvl[(size_t)b * (T + 1) + s] + base;
      float a = f.uval[((size_t)b * (T + 1) + s) * C + c];
      if (emit) {
        // cum[t_ref] - cum[s]: score rows s .. t_ref-1
        double d = 0.0;
        for (int u = s; u < t_ref; ++u) d += (double)em_b[(size_t)u * C + c];
        a += (float)(d * kLog2eD);
      } else {
        a -= (cum_b[(size_t)s * C + c] - cref[c]) * kLog2e;
      }
      if (f.ps != nullptr) a += f.ps[(size_t)b * (f.pseq ? (size_t)f.pseq : (size_t)T * C) + (size_t)s * C + c] * kLog2e;
      const int k0 = t_ref - s + 1, k1 = min(Kmax, len - s);
      float sk0 = 0.0f, sk1 = 0.0f;
#pragma unroll 4
      for (int k = k0; k <= k1; ++k) {
        const int i = s + k - t_lo;
        const float dk = DBL ? dbl[(k - 1) * C + c] : f.db[(size_t)(K == 1 ? 0 : min(k, K - 1)) * C + c] * kLog2e;
        const float y = (float)(al + lvs[i]) + ((a + ew[i * C + c]) + dk);
        if (k & 1) sk1 += exp2_hw(y);
        else sk0 += exp2_hw(y);
      }
      acc += (double)(sk0 + sk1);
    }
  }
  for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double cov = 0.0;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) cov += red[i];
    double* fj = f.mframe + (size_t)b * f.P + j;
    if (j == 0) cov *= *fj;  // start sums are in the chunk frame
    if (cov > 0.5 && cov < 2.0) *fj /= cov;
  }
}

template <bool DBL>
hipError_t launch_coverage(const Plan& pl, const FusedParams& f, hipStream_t s) {
  const size_t lds = coverage_lds(pl.C, pl.Kmax, DBL);
  const hipError_t e =
      hipFuncSetAttribute((const void*)coverage_kernel<DBL>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(coverage_kernel<DBL>, dim3(pl.P, pl.B), dim3(1024), lds, s, f);
  return hipSuccess;
}

// ---- rows: grad_cum / projections ----
__global__ void fused_rows_kernel(FusedParams f) {
  const int b = blockIdx.y;
  const int C = f.C, T = f.T, Lc = f.Lc, Kmax = f.Kmax;
  const int len = flen(f.lengths, b, T);
  const float g = f.grad_output[b];
  const size_t n = (size_t)(T + 1) * C;
  // entry idx = (t, c) of row t, with its own-row end sum eo, start sum so and chunk factor fj
  // (loaded by the caller)
  auto row = [&](int t, int c, size_t o, float eo, float so, double fj) {
    float E = 0.0f, S = 0.0f;
    if (t <= len) {
      if (t > 0) {
        double e = fj * (double)eo;
        const int j = fchunk(t, len, Lc);
        const int d = t - j * Lc;  // rows j*Lc .. j*Lc+Kmax-1 also take chunk j-1's halo
        if (f.halo != nullptr && j >= 1 && d < Kmax)
          e += fscale(f, b, j - 1) * (double)f.halo[(((size_t)b * f.P + j - 1) * Kmax + d) * C + c];
        E = (float)e;
      }
      if (t < len) S = (float)(fj * (double)so);
    }
    if (f.accum) {
      // window of the bounded-memory backward: rows of the full tensors (their
      // strides); rows at the window's edges take parts from two windows
      const size_t xo = (size_t)b * f.xseq + (size_t)t * C + c, po = (size_t)b * f.pseq + (size_t)t * C + c;
      f.grad_cum[xo] += g * (E - S);
      if (f.grad_ps != nullptr && t < T) f.grad_ps[po] += g * S;
      if (f.grad_pe != nullptr && t >= 1) f.grad_pe[po - C] += g * E;
      return;
    }
    if (!f.shift) f.grad_cum[o] = g * (E - S);
    else if (t >= 1) f.grad_cum[((size_t)b * T + t - 1) * C + c] = g * (E - S);
    if (f.grad_ps != nullptr && t < T) f.grad_ps[((size_t)b * T + t) * C + c] = g * S;
    if (f.grad_pe != nullptr && t >= 1) f.grad_pe[((size_t)b * T + t - 1) * C + c] = g * E;
  };
  // four entries per thread loaded before any is used (every load is in bounds: t <= T,
  // and the chunk index is clamped to the sequence's chunks)
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; idx + 3 * stride < n; idx += 4 * stride) {
    int t[4], c[4];
    size_t o[4];
    float eo[4], so[4];
    double fj[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const size_t id = idx + u * stride;
      t[u] = (int)(id / C);
      c[u] = (int)(id % C);
      o[u] = ((size_t)b * (T + 1) + t[u]) * C + c[u];
      eo[u] = f.e_own[o[u]];
      so[u] = f.s_out[o[u]];
      fj[u] = fscale(f, b, fchunk(t[u], len, Lc));
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) row(t[u], c[u], o[u], eo[u], so[u], fj[u]);
  }
  for (; idx < n; idx += stride) {
    const int t = (int)(idx / C), c = (int)(idx % C);
    const size_t o = ((size_t)b * (T + 1) + t) * C + c;
    row(t, c, o, f.e_own[o], f.s_out[o], fscale(f, b, fchunk(t, len, Lc)));
  }
}

// ---- transitions: one block per (sequence, row block); rows staged kGRows at a time ----
// Thread i of the block takes the (source, destination) pairs i, i+nt, ... (NPT
// of them); the block has about C*C/NPT threads.
//
// With x = alpha-hat[t,c'] + tr[c',c] + log2 S[t,c] - u[t,c] the term is 2^x.
// When every column's transition range (max - min over sources) is <= 30 the
// block uses the factorised form 2^x = A[t,c'] * W[t,c] * E[c',c] with
// A = 2^alpha-hat (<= 1), W = 2^(log2 S - u + cm[c]), E = 2^(tr - cm[c]) (<= 1),
// cm[c] the column maximum: u >= cm[c] - range, so W <= S * 2^30, and an A that
// underflows drops a term below 2^-96.  The row loop is then one FMA per pair
// (the sum over rows of A * W, times E at the end) instead of an exponential.
constexpr int kGRows = 64;

template <int NPT>
__global__ void __launch_bounds__(1024) trans_grad_kernel(FusedParams f) {
  extern __shared__ __align__(16) char smem[];
  const int C = f.C, T = f.T, Lc = f.Lc;
  const int b = blockIdx.y, blk = blockIdx.x;
  const int nt = blockDim.x;
  const int len = flen(f.lengths, b, T);
  const int NP = C * C;
  float* ah = reinterpret_cast<float*>(smem);  // [row][c_src] alpha-hat, or A
  float* vq = ah + kGRows * C;                 // [row][c_dst] log2 S - u, or W
  float* fs = vq + kGRows * C;                 // [row] chunk factor of the row's start
  float* cm = fs + kGRows;                     // [c_dst] column maximum of the transitions
  bool wide = false;
  for (int c = threadIdx.x; c < C; c += nt) {
    float hi = kMinusInf, lo = -kMinusInf;
    for (int cs = 0; cs < C; ++cs) {
      const float v = f.trans[(size_t)cs * C + c] * kLog2e;
      hi = fmax2(hi, v);
      lo = fmin(lo, v);
    }
    cm[c] = hi;
    wide = wide || !(hi - lo <= 30.0f);
  }
  const bool fact = !__syncthreads_or(wide);
  float tr2[NPT];
  int cs_[NPT], cd_[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int pr = threadIdx.x + nt * i;
    const int pp = pr < NP ? pr : 0;  // surplus slots repeat pair 0 and are not stored
    cs_[i] = pp / C;
    cd_[i] = pp % C;
    tr2[i] = f.trans[pp] * kLog2e;
  }
  float a32[NPT];
  double a64[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    a32[i] = 0.0f;
    a64[i] = 0.0;
  }
  // starts t in [lo, hi) of this block (t < len)
  const int lo = blk * f.GTB;
  const int hi = min(lo + f.GTB, len);
  for (int tb = lo; tb < hi; tb += kGRows) {
    const int nr = min(kGRows, hi - tb);
    __syncthreads();
    if (threadIdx.x < nr) fs[threadIdx.x] = (float)fscale(f, b, fchunk(tb + threadIdx.x, len, Lc));
    __syncthreads();
    const size_t o0 = ((size_t)b * (T + 1) + tb) * C;
    for (int i = threadIdx.x; i < nr * C; i += nt) {
      const float S = fs[i / C] * f.s_out[o0 + i];
      const float v = (S > 0.0f ? log2_hw(S) : kMinusInf) - f.uval[o0 + i];
      if (fact) {
        ah[i] = exp2_hw(f.aval[o0 + i]);
        vq[i] = exp2_hw(v + cm[i % C]);
      } else {
        ah[i] = f.aval[o0 + i];
        vq[i] = v;
      }
    }
    __syncthreads();
    if (fact) {
#pragma unroll 4
      for (int r = 0; r < nr; ++r) {
        const float* ar = ah + r * C;
        const float* vr = vq + r * C;
#pragma unroll
        for (int i = 0; i < NPT; ++i) a32[i] = fmaf(ar[cs_[i]], vr[cd_[i]], a32[i]);
      }
    } else {
#pragma unroll 4
      for (int r = 0; r < nr; ++r) {
        const float* ar = ah + r * C;
        const float* vr = vq + r * C;
#pragma unroll
        for (int i = 0; i < NPT; ++i) a32[i] += exp2_hw((ar[cs_[i]] + tr2[i]) + vr[cd_[i]]);
      }
    }
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
      a64[i] += (double)a32[i];
      a32[i] = 0.0f;
    }
  }
  double* out = f.tr_part + ((size_t)b * f.GNB + blk) * NP;
#pragma unroll
  for (int i = 0; i < NPT; ++i)
    if (threadIdx.x + nt * i < NP) out[threadIdx.x + nt * i] = fact ? a64[i] * exp2((double)(tr2[i] - cm[cd_[i]])) : a64[i];
}

// ---- shared gradients: one wavefront per output element, fixed summation order ----
__global__ void __launch_bounds__(256) fused_shared_kernel(FusedParams f) {
  const int C = f.C, K = f.K, Kmax = f.Kmax, T = f.T;
  const int n_tr = C * C, n_db = K * C;
  const int idx = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (idx >= n_tr + n_db) return;
  // the lane's partials in a fixed order, eight loaded at once
  double acc = 0.0;
  auto sum_parts = [&](int nparts, auto term) {
    int j = lane;
    for (; j + 7 * 64 < nparts; j += 8 * 64) {
      double v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = term(j + u * 64);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += v[u];
    }
    for (; j < nparts; j += 64) acc += term(j);
  };
  if (idx < n_tr) {
    sum_parts(f.B * f.GNB, [&](int j) { return (double)f.grad_output[j / f.GNB] * f.tr_part[(size_t)j * n_tr + idx]; });
  } else {
    const int e = idx - n_tr;
    const int k = e / C, c = e % C;
    // durations mapping to duration-bias row k: k itself (K >= 2, k >= 1) or 1 (K == 1)
    const int dur = (K == 1) ? 1 : k;
    if (dur >= 1 && dur <= Kmax) {
      sum_parts(f.B * f.P, [&](int it) {
        const int b = it / f.P, j = it % f.P;
        const int len = flen(f.lengths, b, T);
        if (j > (len > 0 ? (len - 1) / f.Lc : 0)) return 0.0;  // empty chunk
        return (double)f.grad_output[b] * fscale(f, b, j) * f.db_part[((size_t)it * Kmax + dur - 1) * C + c];
      });
    }
  }
  for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (lane == 0) {
    float* out = idx < n_tr ? f.grad_tr + idx : f.grad_db + (idx - n_tr);
    *out = f.accum ? *out + (float)acc : (float)acc;
  }
}

}  // namespace

template <int CP>
int launch_u_cp(const FusedParams& f, dim3 grid, size_t lds, hipStream_t s) {
  const hipError_t e = hipFuncSetAttribute((const void*)u_rows_kernel<CP>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(u_rows_kernel<CP>, grid, dim3(256), lds, s, f);
  return hipSuccess;
}

int launch_u_rows(const Plan& pl, const FusedParams& f, hipStream_t s) {
  const int CP = pl.C <= 8 ? 8 : pl.C <= 16 ? 16 : pl.C <= 32 ? 32 : pl.C <= 64 ? 64 : 128;
  if (pl.C > 128) return (int)hipErrorInvalidValue;
  const size_t lds = sizeof(float) * ((size_t)pl.C * pl.C + (size_t)kURows * CP + 2 * (size_t)pl.C);
  const dim3 grid((pl.T + 1 + kURows - 1) / kURows, pl.B);
  TimedLaunch tl(kKURows, s);
  int e;
  switch (CP) {
    case 8: e = launch_u_cp<8>(f, grid, lds, s); break;
    case 16: e = launch_u_cp<16>(f, grid, lds, s); break;
    case 32: e = launch_u_cp<32>(f, grid, lds, s); break;
    case 64: e = launch_u_cp<64>(f, grid, lds, s); break;
    default: e = launch_u_cp<128>(f, grid, lds, s); break;
  }
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

template <int NPT>
int launch_trans_grad(const Plan& pl, const FusedParams& f, hipStream_t s) {
  const size_t lds = sizeof(float) * (2 * (size_t)kGRows * pl.C + kGRows + pl.C);
  const hipError_t e = hipFuncSetAttribute((const void*)trans_grad_kernel<NPT>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  const int np = pl.C * pl.C;
  int nt = (np + NPT - 1) / NPT;
  nt = std::max(64, std::min(1024, (nt + 63) / 64 * 64));
  hipLaunchKernelGGL(trans_grad_kernel<NPT>, dim3(pl.GNB, pl.B), dim3(nt), lds, s, f);
  return hipSuccess;
}

int launch_fused_finalize(const Plan& pl, const FusedParams& f, hipStream_t s) {
  // pairs per thread: with 256 threads up to 16; above C*C = 4096 (C <= 128) 16 pairs
  // per thread on up to 1024 threads
  const int np = pl.C * pl.C;
  const int npt = np <= 4096 ? (np + 255) / 256 : 16;
  if (np > 16 * 1024) return (int)hipErrorInvalidValue;
  {
    const int n = pl.B * pl.P;
    hipLaunchKernelGGL(frame_scale_kernel, dim3((n + 255) / 256), dim3(256), 0, s, f);
  }
  const char* cenv = getenv("TSM_COVERAGE");  // diagnostics: =0 skips the coverage correction
  if (cenv == nullptr || strcmp(cenv, "0") != 0) {
    TimedLaunch tl(kKCoverage, s);
    // fused plans have C <= 64 and Kmax <= 512: ew and the levels always fit LDS
    const hipError_t e = coverage_lds(pl.C, pl.Kmax, true) <= 160 * 1024 ? launch_coverage<true>(pl, f, s)
                                                                           : launch_coverage<false>(pl, f, s);
    if (e != hipSuccess) return e;
  }
  int gx = (int)(((size_t)(pl.T + 1) * pl.C + 255) / 256);
  if (gx > 4096) gx = 4096;
  {
    TimedLaunch tl(kKFusedRows, s);
    hipLaunchKernelGGL(fused_rows_kernel, dim3(gx, pl.B), dim3(256), 0, s, f);
  }
  {
    TimedLaunch tl(kKTransGrad, s);
    int e;
    if (npt <= 1) e = launch_trans_grad<1>(pl, f, s);
    else if (npt <= 2) e = launch_trans_grad<2>(pl, f, s);
    else if (npt <= 3) e = launch_trans_grad<3>(pl, f, s);
    else if (npt <= 4) e = launch_trans_grad<4>(pl, f, s);
    else if (npt <= 8) e = launch_trans_grad<8>(pl, f, s);
    else e = launch_trans_grad<16>(pl, f, s);
    if (e != hipSuccess) return e;
  }
  {
    TimedLaunch tl(kKFusedShared, s);
    const int n = pl.C * pl.C + pl.K * pl.C;
    hipLaunchKernelGGL(fused_shared_kernel, dim3((n + 3) / 4), dim3(256), 0, s, f);
  }
  return hipGetLastError();
}

}  // namespace tsm
