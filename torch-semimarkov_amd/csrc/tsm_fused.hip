// Backward with the segment marginals fused into the register-resident beta
// scan (tsm_fastscan.hpp, MARG): the row passes around it.
//
//   u pass      u[t,c] = log2 sum_c' 2^(alpha-hat[t,c'] + trans[c',c] log2 e), the
//               forward side of a segment starting at t with label c (the scan
//               reads one value per step instead of redoing the label mix);
//   scan        per chunk j, in its own frame: end sums e_own / halo, start sums
//               s_out, duration sums db_part, frame estimate mframe[j];
//   rows        grad_cum / grad_proj from E and S, each chunk's values times
//               f_j = 2^(mframe[j] + offs[j]) (offs: the chunk's verified
//               level offset), which takes them to probabilities;
//   transitions G[c',c] = sum_t 2^(alpha-hat[t,c'] + trans[c',c] log2 e - u[t,c]) S[t,c]
//               (the softmax weight of source c' times the start sum), per row
//               block in fp64;
//   shared      grad_db = sum_j f_j db_part[j], grad_tr = sum of the row blocks,
//               both weighted by grad_output, in a fixed order.
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
constexpr int kURows = 64;

__global__ void __launch_bounds__(256) u_rows_kernel(FusedParams f) {
  extern __shared__ __align__(16) char smem[];
  const int C = f.C, T = f.T;
  const int b = blockIdx.y;
  const int len = flen(f.lengths, b, T);
  const int t0 = blockIdx.x * kURows;
  if (t0 > len) return;
  const int nr = min(kURows, len + 1 - t0);
  float* tr2 = reinterpret_cast<float*>(smem);  // [c_src][c_dst], log2 units
  float* ah = tr2 + C * C;                       // [row][c]
  for (int i = threadIdx.x; i < C * C; i += blockDim.x) tr2[i] = f.trans[i] * kLog2e;
  const float* av = f.aval + ((size_t)b * (T + 1) + t0) * C;
  for (int i = threadIdx.x; i < nr * C; i += blockDim.x) ah[i] = av[i];
  __syncthreads();
  float* uo = f.uval + ((size_t)b * (T + 1) + t0) * C;
  for (int i = threadIdx.x; i < nr * C; i += blockDim.x) {
    const int r = i / C, c = i % C;
    const float* a = ah + r * C;
    float m = kMinusInf;
    for (int cs = 0; cs < C; ++cs) m = fmax2(m, a[cs] + tr2[cs * C + c]);
    float s = 0.0f;
    for (int cs = 0; cs < C; ++cs) s += exp2_hw((a[cs] + tr2[cs * C + c]) - m);
    uo[i] = m + log2_hw(s);
  }
}

// ---- rows: grad_cum / projections ----
__global__ void fused_rows_kernel(FusedParams f) {
  const int b = blockIdx.y;
  const int C = f.C, T = f.T, Lc = f.Lc, Kmax = f.Kmax;
  const int len = flen(f.lengths, b, T);
  const float g = f.grad_output[b];
  const size_t n = (size_t)(T + 1) * C;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (size_t)gridDim.x * blockDim.x) {
    const int t = (int)(idx / C), c = (int)(idx % C);
    const size_t o = ((size_t)b * (T + 1) + t) * C + c;
    float E = 0.0f, S = 0.0f;
    if (t <= len) {
      const int j = fchunk(t, len, Lc);
      const double fj = fscale(f, b, j);
      if (t > 0) {
        double e = fj * (double)f.e_own[o];
        const int d = t - j * Lc;  // rows j*Lc .. j*Lc+Kmax-1 also take chunk j-1's halo
        if (j >= 1 && d < Kmax) e += fscale(f, b, j - 1) * (double)f.halo[(((size_t)b * f.P + j - 1) * Kmax + d) * C + c];
        E = (float)e;
      }
      if (t < len) S = (float)(fj * (double)f.s_out[o]);
    }
    f.grad_cum[o] = g * (E - S);
    if (f.grad_ps != nullptr && t < T) f.grad_ps[((size_t)b * T + t) * C + c] = g * S;
    if (f.grad_pe != nullptr && t >= 1) f.grad_pe[((size_t)b * T + t - 1) * C + c] = g * E;
  }
}

// ---- transitions: one block per (sequence, row block); rows staged kGRows at a time ----
// Thread i of 256 takes the (source, destination) pairs i, i+256, ... (NPT of them).
constexpr int kGRows = 128;

template <int NPT>
__global__ void __launch_bounds__(256) trans_grad_kernel(FusedParams f) {
  extern __shared__ __align__(16) char smem[];
  const int C = f.C, T = f.T, Lc = f.Lc;
  const int b = blockIdx.y, blk = blockIdx.x;
  const int len = flen(f.lengths, b, T);
  const int NP = C * C;
  float* ah = reinterpret_cast<float*>(smem);  // [row][c_src] alpha-hat
  float* vq = ah + kGRows * C;                 // [row][c_dst] log2 S - u
  float tr2[NPT];
  int cs_[NPT], cd_[NPT];
#pragma unroll
  for (int i = 0; i < NPT; ++i) {
    const int pr = threadIdx.x + 256 * i;
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
    for (int i = threadIdx.x; i < nr * C; i += blockDim.x) {
      const int r = i / C, c = i % C, t = tb + r;
      const size_t o = ((size_t)b * (T + 1) + t) * C + c;
      ah[i] = f.aval[o];
      const float S = (float)(fscale(f, b, fchunk(t, len, Lc)) * (double)f.s_out[o]);
      vq[i] = (S > 0.0f ? log2_hw(S) : kMinusInf) - f.uval[o];
    }
    __syncthreads();
    for (int r = 0; r < nr; ++r) {
      const float* ar = ah + r * C;
      const float* vr = vq + r * C;
#pragma unroll
      for (int i = 0; i < NPT; ++i) a32[i] += exp2_hw((ar[cs_[i]] + tr2[i]) + vr[cd_[i]]);
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
    if (threadIdx.x + 256 * i < NP) out[threadIdx.x + 256 * i] = a64[i];
}

// ---- shared gradients: one wavefront per output element, fixed summation order ----
__global__ void __launch_bounds__(256) fused_shared_kernel(FusedParams f) {
  const int C = f.C, K = f.K, Kmax = f.Kmax, T = f.T;
  const int n_tr = C * C, n_db = K * C;
  const int idx = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (idx >= n_tr + n_db) return;
  double acc = 0.0;
  if (idx < n_tr) {
    const int nparts = f.B * f.GNB;
    for (int j = lane; j < nparts; j += 64)
      acc += (double)f.grad_output[j / f.GNB] * f.tr_part[(size_t)j * n_tr + idx];
  } else {
    const int e = idx - n_tr;
    const int k = e / C, c = e % C;
    // durations mapping to duration-bias row k: k itself (K >= 2, k >= 1) or 1 (K == 1)
    const int dur = (K == 1) ? 1 : k;
    if (dur >= 1 && dur <= Kmax) {
      const int nparts = f.B * f.P;
      for (int it = lane; it < nparts; it += 64) {
        const int b = it / f.P, j = it % f.P;
        const int len = flen(f.lengths, b, T);
        if (j > (len > 0 ? (len - 1) / f.Lc : 0)) continue;  // empty chunk
        acc += (double)f.grad_output[b] * fscale(f, b, j) * f.db_part[((size_t)it * Kmax + dur - 1) * C + c];
      }
    }
  }
  for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (lane == 0) {
    if (idx < n_tr) f.grad_tr[idx] = (float)acc;
    else f.grad_db[idx - n_tr] = (float)acc;
  }
}

}  // namespace

int launch_u_rows(const Plan& pl, const FusedParams& f, hipStream_t s) {
  const size_t lds = sizeof(float) * ((size_t)pl.C * pl.C + (size_t)kURows * pl.C);
  TimedLaunch tl(kKURows, s);
  hipLaunchKernelGGL(u_rows_kernel, dim3((pl.T + 1 + kURows - 1) / kURows, pl.B), dim3(256), lds, s, f);
  return hipGetLastError();
}

template <int NPT>
void launch_trans_grad(const Plan& pl, const FusedParams& f, hipStream_t s) {
  const size_t lds = sizeof(float) * 2 * (size_t)kGRows * pl.C;
  hipLaunchKernelGGL(trans_grad_kernel<NPT>, dim3(pl.GNB, pl.B), dim3(256), lds, s, f);
}

int launch_fused_finalize(const Plan& pl, const FusedParams& f, hipStream_t s) {
  const int npt = (pl.C * pl.C + 255) / 256;
  if (npt > 16) return (int)hipErrorInvalidValue;
  {
    const int n = pl.B * pl.P;
    hipLaunchKernelGGL(frame_scale_kernel, dim3((n + 255) / 256), dim3(256), 0, s, f);
  }
  int gx = (int)(((size_t)(pl.T + 1) * pl.C + 255) / 256);
  if (gx > 4096) gx = 4096;
  {
    TimedLaunch tl(kKFusedRows, s);
    hipLaunchKernelGGL(fused_rows_kernel, dim3(gx, pl.B), dim3(256), 0, s, f);
  }
  {
    TimedLaunch tl(kKTransGrad, s);
    if (npt <= 1) launch_trans_grad<1>(pl, f, s);
    else if (npt <= 2) launch_trans_grad<2>(pl, f, s);
    else if (npt <= 3) launch_trans_grad<3>(pl, f, s);
    else if (npt <= 4) launch_trans_grad<4>(pl, f, s);
    else if (npt <= 8) launch_trans_grad<8>(pl, f, s);
    else launch_trans_grad<16>(pl, f, s);
  }
  {
    TimedLaunch tl(kKFusedShared, s);
    const int n = pl.C * pl.C + pl.K * pl.C;
    hipLaunchKernelGGL(fused_shared_kernel, dim3((n + 3) / 4), dim3(256), 0, s, f);
  }
  return hipGetLastError();
}

}  // namespace tsm
