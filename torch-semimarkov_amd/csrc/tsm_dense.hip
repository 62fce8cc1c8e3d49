// Duration-dependent transitions (trows, C, C): transition tables, segment
// marginals and gradients, for gfx950.  The scans are in tsm_dense_scan.hpp
// (instantiated in tsm_dense_f.hip / tsm_dense_b.hip).
//
// Marginals.  For a segment starting at s with duration k, label c and
// predecessor c' (reference streaming/pytorch_reference.py:425-499):
//   m(s,k,c',c) = exp( alpha[s,c'] + trans[k][c',c] + seg(s,k,c) + beta[s+k,c] - logZ )
// and, with P(s,k,c) = sum_{c'} m,
//   d cum[s+k,c] += P, d cum[s,c] -= P, d db[min(k,K-1),c] += P,
//   d proj_start[s,c] += P, d proj_end[s+k-1,c] += P, d trans[k][c',c] += m.
// Every (s,k,c',c) term is one exponential; nothing factors.
//
// One workgroup handles the TB start positions of one block of one sequence,
// every duration and label pair.  Lanes are laid out as label groups of G
// lanes: group g serves destination labels c = g, g+NG, ..., lane l source
// labels c' = l, l+G, ...; P(s,k,c) is a DPP sum over the group.  Durations are
// the outer loop, so the transition gradient of one duration accumulates in
// registers and is folded into the block's fp64 partials every 64 positions; start
// and end sums accumulate in LDS rows owned by one lane each, and leave the
// block in the layout of the other marginal kernels (own end rows, a halo of
// Kmax rows for the next block, fp64 per-block partials), so the same
// finalize kernels produce the gradients.  No atomics.

#include "tsm_dense_scan.hpp"

namespace tsm {
namespace dense {

int launch_dense_fwd(const Plan& pl, const ScanParams& p, int semiring, hipStream_t s);
int launch_dense_bwd(const Plan& pl, const ScanParams& p, int semiring, hipStream_t s);

namespace {

constexpr int kMaxCPG = 8;  // destination labels per lane group (C <= 128 with 16 groups)
constexpr int kMaxCPL = 2;  // source labels per lane (C <= 128 with 64 lanes)

// trf[k-1][c_dst][c_src] and trb[k-1][c_src][c_dst] = transition[k][c_src][c_dst] * log2(e),
// k = 1..Kmax (the durations the recursion uses).
__global__ void dense_prep_kernel(const float* tr, int C, int Kmax, float* trf, float* trb) {
  const size_t n = (size_t)Kmax * C * C;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (size_t)gridDim.x * blockDim.x) {
    const size_t r = idx / ((size_t)C * C);
    const int a = (int)((idx / C) % C), bb = (int)(idx % C);
    const float* m = tr + (r + 1) * C * C;
    trf[idx] = m[(size_t)bb * C + a] * kLog2e;
    trb[idx] = m[(size_t)a * C + bb] * kLog2e;
  }
}

__device__ inline int dlen(const int64_t* lengths, int b, int T) {
  int64_t L = lengths[b];
  if (L < 0) L = 0;
  if (L > T) L = T;
  return (int)L;
}

template <int G>
__global__ void __launch_bounds__(1024) dense_marginal_kernel(MargParams q) {
  extern __shared__ __align__(16) char smem[];
  const int blk = blockIdx.x % q.NB;
  const int b = blockIdx.x / q.NB;
  const int C = q.C, Kmax = q.Kmax, K = q.K, T = q.T, TB = q.TB;
  const int len = dlen(q.lengths, b, T);
  const int t0 = blk * TB;
  const int tid = threadIdx.x, NT = blockDim.x;
  const int NG = NT / G, g = tid / G, l = tid % G;
  float* e_own_b = q.e_own + (size_t)b * (T + 1) * C;
  double* dbp = q.db_part + ((size_t)b * q.NB + blk) * Kmax * C;
  double* trp = q.tr_part + ((size_t)b * q.NB + blk) * Kmax * C * C;
  if (t0 >= len) {
    // no starts here: zero this block's partials (summed over all blocks) and
    // the end-sum row at len when the block begins there
    for (int idx = tid; idx < Kmax * C; idx += NT) dbp[idx] = 0.0;
    for (size_t idx = tid; idx < (size_t)Kmax * C * C; idx += NT) trp[idx] = 0.0;
    if (t0 == len)
      for (int cc = tid; cc < C; cc += NT) e_own_b[(size_t)len * C + cc] = 0.0f;
    return;
  }
  const int t1 = min(t0 + TB, len);
  const bool has_ps = q.ps != nullptr, has_pe = q.pe != nullptr;
  const DenseMargLds Ly = dense_marg_lds_layout(C, Kmax, TB);
  float* sacc = reinterpret_cast<float*>(smem + Ly.sacc);
  float* eacc = reinterpret_cast<float*>(smem + Ly.eacc);
  for (int idx = tid; idx < TB * C; idx += NT) sacc[idx] = 0.0f;
  for (int idx = tid; idx < (TB + Kmax) * C; idx += NT) eacc[idx] = 0.0f;
  __syncthreads();

  const float* cum_b = q.cum + (size_t)b * (T + 1) * C;
  const float* ps_b = has_ps ? q.ps + (size_t)b * T * C : nullptr;
  const float* pe_b = has_pe ? q.pe + (size_t)b * T * C : nullptr;
  const float* av_b = q.aval + (size_t)b * (T + 1) * C;
  const double* al_b = q.alvl + (size_t)b * (T + 1);
  const float* bv_b = q.bval + (size_t)b * (T + 1) * C;
  const double* bl_b = q.blvl + (size_t)b * (T + 1);
  const double z2 = q.z2[b];

  for (int k = 1; k <= Kmax; ++k) {
    const int di = k < K - 1 ? k : K - 1;
    const float* trk = q.trx + (size_t)(k - 1) * C * C;
    // fp32 partials of this lane's transition-gradient entries, folded into the
    // block's fp64 partials (owned by this lane, zeroed here) every 64 positions
    float tpart[kMaxCPG][kMaxCPL];
    float dacc[kMaxCPG], dbk[kMaxCPG];
    double* trk_part = trp + (size_t)(k - 1) * C * C;
#pragma unroll
    for (int gi = 0; gi < kMaxCPG; ++gi) {
      const int cd = g + NG * gi;
      dacc[gi] = 0.0f;
      dbk[gi] = (cd < C) ? q.db[(size_t)di * C + cd] * kLog2e : 0.0f;
#pragma unroll
      for (int li = 0; li < kMaxCPL; ++li) {
        const int cp = l + G * li;
        tpart[gi][li] = 0.0f;
        if (cd < C && cp < C) trk_part[(size_t)cp * C + cd] = 0.0;
      }
    }
    auto fold = [&]() {
#pragma unroll
      for (int gi = 0; gi < kMaxCPG; ++gi) {
        const int cd = g + NG * gi;
#pragma unroll
        for (int li = 0; li < kMaxCPL; ++li) {
          const int cp = l + G * li;
          if (cd < C && cp < C) trk_part[(size_t)cp * C + cd] += (double)tpart[gi][li];
          tpart[gi][li] = 0.0f;
        }
      }
    };
    // starts whose segment of duration k ends inside the sequence
    const int s_hi = min(t1, len - k + 1);
    for (int s = t0; s < s_hi; ++s) {
      const float lv = (float)(al_b[s] + bl_b[s + k] - z2);
      const float* ar = av_b + (size_t)s * C;
      const float* cs_row = cum_b + (size_t)s * C;
      const float* ce_row = cum_b + (size_t)(s + k) * C;
      const float* be_row = bv_b + (size_t)(s + k) * C;
      float av[kMaxCPL];
#pragma unroll
      for (int li = 0; li < kMaxCPL; ++li) {
        const int cp = l + G * li;
        av[li] = (cp < C) ? ar[cp] : 0.0f;
      }
#pragma unroll
      for (int gi = 0; gi < kMaxCPG; ++gi) {
        const int cd = g + NG * gi;
        if (cd < C) {
          float rest = dbk[gi] + be_row[cd] + lv;
          if (has_ps) rest += ps_b[(size_t)s * C + cd] * kLog2e;
          if (has_pe) rest += pe_b[(size_t)(s + k - 1) * C + cd] * kLog2e;
          const float qq = fmaf(ce_row[cd] - cs_row[cd], kLog2e, rest);
          const float* trow = trk + (size_t)cd * C;
          float psum = 0.0f;
#pragma unroll
          for (int li = 0; li < kMaxCPL; ++li) {
            const int cp = l + G * li;
            if (cp < C) {
              const float e = exp2_hw((av[li] + trow[cp]) + qq);
              tpart[gi][li] += e;
              psum += e;
            }
          }
          const float P = group_sum<G>(psum);
          if (l == 0) {
            sacc[(s - t0) * C + cd] += P;
            eacc[(s + k - t0) * C + cd] += P;
            dacc[gi] += P;
          }
        }
      }
      if (((s - t0) & 63) == 63) fold();
    }
    fold();
#pragma unroll
    for (int gi = 0; gi < kMaxCPG; ++gi) {
      const int cd = g + NG * gi;
      if (cd < C && l == 0) dbp[(size_t)(k - 1) * C + cd] = (double)dacc[gi];
    }
  }
  __syncthreads();
  for (int idx = tid; idx < (t1 - t0) * C; idx += NT)
    q.s_out[((size_t)b * (T + 1) + t0) * C + idx] = sacc[idx];
  // end rows: (t0, t0+TB) own, [t0+TB, t0+TB+Kmax) halo of the next block; row t0 is 0
  for (int idx = tid; idx < (TB + Kmax) * C; idx += NT) {
    const int i = idx / C, cc = idx % C;
    const int r = t0 + i;
    if (r > len) continue;
    if (i < TB) e_own_b[(size_t)r * C + cc] = eacc[idx];
    else q.halo[(((size_t)b * q.NB + blk) * Kmax + (i - TB)) * C + cc] = eacc[idx];
  }
}

template <int G>
int launch_dmarg(const Plan& pl, const MargParams& q, hipStream_t st) {
  auto k = dense_marginal_kernel<G>;
  hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl.dmarg_lds);
  if (e != hipSuccess) return e;
  {
    TimedLaunch tl(kKMarginal, st);
    hipLaunchKernelGGL(k, dim3(pl.B * pl.DNB), dim3(pl.DNTM), pl.dmarg_lds, st, q);
  }
  return hipGetLastError();
}

}  // namespace
}  // namespace dense

int launch_dense_prep(const Plan& pl, const float* trans, float* trf, float* trb, hipStream_t s) {
  const size_t n = (size_t)pl.Kmax * pl.C * pl.C;
  int g = (int)((n + 255) / 256);
  if (g > 4096) g = 4096;
  {
    TimedLaunch tl(kKTransPrep, s);
    hipLaunchKernelGGL(dense::dense_prep_kernel, dim3(g), dim3(256), 0, s, trans, pl.C, pl.Kmax, trf, trb);
  }
  return hipGetLastError();
}

int launch_dense_scan(const Plan& pl, const ScanParams& p, int semiring, bool forward, hipStream_t s) {
  return forward ? dense::launch_dense_fwd(pl, p, semiring, s) : dense::launch_dense_bwd(pl, p, semiring, s);
}

int launch_dense_marginals(const Plan& pl, const MargParams& q, hipStream_t s) {
  switch (pl.DG) {
    case 1: return dense::launch_dmarg<1>(pl, q, s);
    case 2: return dense::launch_dmarg<2>(pl, q, s);
    case 4: return dense::launch_dmarg<4>(pl, q, s);
    case 8: return dense::launch_dmarg<8>(pl, q, s);
    case 16: return dense::launch_dmarg<16>(pl, q, s);
    case 32: return dense::launch_dmarg<32>(pl, q, s);
    case 64: return dense::launch_dmarg<64>(pl, q, s);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace tsm
