// Segment marginals and gradients (after both scans), for gfx950.
//
// For a segment starting at t with duration k and label c (any predecessor):
//   P(t,k,c) = exp( u[t,c] + seg(t,k,c) + beta[t+k,c] - logZ ),
//   u[t,c]   = LSE_{c'} alpha[t,c'] + trans[c',c]
// and the reference's gradients (streaming/pytorch_reference.py:456-499) are
//   d cum[t+k,c] += P, d cum[t,c] -= P, d db[min(k,K-1),c] += P,
//   d proj_start[t,c] += P, d proj_end[t+k-1,c] += P,
//   d trans[c',c] += exp(alpha[t,c'] + trans[c',c] - u[t,c]) * sum_k P(t,k,c).
// (For the max semiring the same formulas with max-alpha/beta give the
// reference's "soft max-marginals", pytorch_reference.py:458-467.)
//
// One workgroup handles TB consecutive start positions of one sequence; all
// blocks are independent.  End sums E[r,c] = sum_k P(r-k,k,c) accumulate in an
// LDS ring and are flushed row by row; rows that belong to the next block
// ("halo", at most Kmax-1 rows) go to a side buffer that the finalize kernel
// adds.  Nothing uses atomics: every output element has exactly one writer.

#include "tsm_device.hpp"
#include "tsm_internal.hpp"

namespace tsm {
namespace {

constexpr double kLog2eM = 1.4426950408889634;  // log2(e) in fp64

constexpr int kTRegMax = 8;  // register accumulators per lane for the transition gradient

__device__ inline int mlen(const int64_t* lengths, int b, int T) {
  int64_t L = lengths[b];
  if (L < 0) L = 0;
  if (L > T) L = T;
  return (int)L;
}

// Block (b, position block blk, label block cbk): start positions
// [t0, t0+TB) of sequence b, destination labels [cb0, cb0+CB).
template <int J>
__global__ void __launch_bounds__(512) marginal_kernel(MargParams q) {
  extern __shared__ __align__(16) char smem[];
  const int cbk = blockIdx.x % q.NCB;
  const int blk = (blockIdx.x / q.NCB) % q.NB;
  const int b = blockIdx.x / (q.NCB * q.NB);
  const int C = q.C, CB = q.CB, Kmax = q.Kmax, RS = q.RS, T = q.T, K = q.K;
  const int cb0 = cbk * CB;
  const int len = mlen(q.lengths, b, T);
  const int t0 = blk * q.TB;
  const int tid = threadIdx.x, NT = blockDim.x;
  const int cl_raw = tid / J, lj = tid % J;
  const bool cval = cl_raw < CB && cb0 + cl_raw < C;
  const int cl = cval ? cl_raw : 0;       // local label
  const int c = cb0 + cl;                 // global label
  const int ncl = min(CB, C - cb0);       // labels in this block
  float* e_own_b = q.e_own + (size_t)b * (T + 1) * C;
  if (t0 >= len) {
    // no starts here: zero this block's gradient partials (they are summed over
    // all blocks) and the end-sum row at len when the block begins there
    double* dbz = q.db_part + ((size_t)b * q.NB + blk) * Kmax * C;
    double* trz = q.tr_part + ((size_t)b * q.NB + blk) * C * C;
    for (int idx = tid; idx < Kmax * ncl; idx += NT) dbz[(size_t)(idx / ncl) * C + cb0 + idx % ncl] = 0.0;
    for (int idx = tid; idx < C * ncl; idx += NT) trz[(size_t)(idx / ncl) * C + cb0 + idx % ncl] = 0.0;
    if (t0 == len)
      for (int i = tid; i < ncl; i += NT) e_own_b[(size_t)len * C + cb0 + i] = 0.0f;
    return;
  }
  const int t1 = min(t0 + q.TB, len);
  const bool has_ps = q.ps != nullptr, has_pe = q.pe != nullptr;

  const MargLds L = marg_lds_layout(C, CB, Kmax, RS, has_pe);
  double* lvb = reinterpret_cast<double*>(smem + L.lvb);
  float* brng = reinterpret_cast<float*>(smem + L.brng);
  float* crng = reinterpret_cast<float*>(smem + L.crng);
  float* prng = reinterpret_cast<float*>(smem + L.prng);
  float* erng = reinterpret_cast<float*>(smem + L.erng);
  float* dbt = reinterpret_cast<float*>(smem + L.dbt);
  float* dacc = reinterpret_cast<float*>(smem + L.dacc);
  float* trt = reinterpret_cast<float*>(smem + L.trt);
  float* row = reinterpret_cast<float*>(smem + L.row);
  float* bk = reinterpret_cast<float*>(smem + L.bk);

  const float* cum_b = q.cum + (size_t)b * (T + 1) * C;
  const float* ps_b = has_ps ? q.ps + (size_t)b * T * C : nullptr;
  const float* pe_b = has_pe ? q.pe + (size_t)b * T * C : nullptr;
  const float* av_b = q.aval + (size_t)b * (T + 1) * C;
  const double* al_b = q.alvl + (size_t)b * (T + 1);
  const float* bv_b = q.bval + (size_t)b * (T + 1) * C;
  const double* bl_b = q.blvl + (size_t)b * (T + 1);
  const double z2 = q.z2[b];
  double* dbp = q.db_part + ((size_t)b * q.NB + blk) * Kmax * C;
  double* trp = q.tr_part + ((size_t)b * q.NB + blk) * C * C;

  // ---- constants, initial rings, zeroed partials (this block's labels) ----
  for (int idx = tid; idx < ncl * (Kmax + 1); idx += NT) {
    const int l = idx / (Kmax + 1), k = idx % (Kmax + 1);
    const int di = k < K - 1 ? k : K - 1;
    dbt[idx] = (k == 0) ? 0.0f : q.db[(size_t)di * C + cb0 + l] * kLog2e;
  }
  for (int idx = tid; idx < ncl * C; idx += NT) {
    const int l = idx / C, cs = idx % C;
    trt[idx] = q.trans[(size_t)cs * C + cb0 + l] * kLog2e;  // [c_dst local][c_src]
  }
  for (int idx = tid; idx < CB * RS; idx += NT) erng[idx] = 0.0f;
  for (int idx = tid; idx < CB * (Kmax + 1); idx += NT) dacc[idx] = 0.0f;
  for (int idx = tid; idx < Kmax * ncl; idx += NT) {
    const int i = idx / ncl, l = idx % ncl;
    const int pos = t0 + 1 + i;  // beta / cum positions [t0+1, t0+Kmax]
    if (pos <= len) {
      brng[l * RS + pos % RS] = bv_b[(size_t)pos * C + cb0 + l];
      crng[l * RS + pos % RS] = cum_b[(size_t)pos * C + cb0 + l];
    }
    const int ppos = t0 + i;  // proj_end positions [t0, t0+Kmax-1]
    if (has_pe && ppos < len) prng[l * RS + ppos % RS] = pe_b[(size_t)ppos * C + cb0 + l] * kLog2e;
    dbp[(size_t)i * C + cb0 + l] = 0.0;
  }
  for (int i = tid; i < Kmax; i += NT) {
    const int pos = t0 + 1 + i;
    if (pos <= len) lvb[pos % RS] = bl_b[pos];
  }
  for (int idx = tid; idx < C * ncl; idx += NT) trp[(size_t)(idx / ncl) * C + cb0 + idx % ncl] = 0.0;
  if (cval && lj == 0) e_own_b[(size_t)t0 * C + c] = 0.0f;

  float tacc[kTRegMax];
#pragma unroll
  for (int r = 0; r < kTRegMax; ++r) tacc[r] = 0.0f;
  __syncthreads();
  // fp32 partial sums are folded into the fp64 block partials every 64 steps
  auto flush_acc = [&]() {
    if (!cval) return;
    float* da = dacc + cl * (Kmax + 1);
    for (int k = 1 + lj; k <= Kmax; k += J) {
      dbp[(size_t)(k - 1) * C + c] += (double)da[k];
      da[k] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < kTRegMax; ++r) {
      const int cs = lj + r * J;
      if (cs < C) trp[(size_t)cs * C + c] += (double)tacc[r];
      tacc[r] = 0.0f;
    }
  };

  const float* br = brng + cl * RS;
  const float* cr = crng + cl * RS;
  const float* pr = prng + cl * RS;
  float* er = erng + cl * RS;
  const float* dr = dbt + cl * (Kmax + 1);
  const float* tr = trt + cl * C;
  for (int t = t0; t < t1; ++t) {
    const int buf = t & 1;
    const int kcap = min(Kmax, len - t);
    // ---- stage per-step shared operands (double buffered) ----
    for (int i = tid; i < C; i += NT) row[buf * C + i] = av_b[(size_t)t * C + i];
    const double al = al_b[t];
    for (int k = tid + 1; k <= kcap; k += NT) {
      int slot = t % RS + k;
      if (slot >= RS) slot -= RS;
      bk[buf * (Kmax + 1) + k] = (float)(al + lvb[slot] - z2);
    }
    // ---- stage the ring entries first needed by step t+1 (position t+1+Kmax,
    //      proj_end position t+Kmax).  With RS >= Kmax+2 their slots are not read
    //      by step t-1, and the barrier below publishes them before step t+1. ----
    {
      const int pos = t + 1 + Kmax;
      if (pos <= len) {
        for (int i = tid; i < ncl; i += NT) {
          brng[i * RS + pos % RS] = bv_b[(size_t)pos * C + cb0 + i];
          crng[i * RS + pos % RS] = cum_b[(size_t)pos * C + cb0 + i];
        }
        if (tid == 0) lvb[pos % RS] = bl_b[pos];
      }
      const int ppos = t + Kmax;
      if (has_pe && ppos < len)
        for (int i = tid; i < ncl; i += NT) prng[i * RS + ppos % RS] = pe_b[(size_t)ppos * C + cb0 + i] * kLog2e;
    }
    __syncthreads();
    const float* rw = row + buf * C;
    const float* bkk = bk + buf * (Kmax + 1);
    // ---- u[t,c] = LSE_{c'} alpha-hat[t,c'] + trans[c',c] ----
    float m = kMinusInf;
    for (int i = lj; i < C; i += J) m = fmax2(m, rw[i] + tr[i]);
    const float M = group_max<J>(m);
    float sm = 0.0f;
    for (int i = lj; i < C; i += J) sm += exp2_hw(rw[i] + tr[i] - M);
    const float S = group_sum<J>(sm);
    const float u2 = M + log2_hw(S);
    const float cur_cum = cum_b[(size_t)t * C + c];
    const float head = u2 + (has_ps ? ps_b[(size_t)t * C + c] * kLog2e : 0.0f);
    // ---- segment marginals P(t,k,c) over durations ----
    const int base = t % RS;
    float sp = 0.0f;
    float* da = dacc + cl * (Kmax + 1);
    for (int k = 1 + lj; k <= kcap; k += J) {
      int slot = base + k;
      if (slot >= RS) slot -= RS;
      float rest = dr[k] + br[slot] + bkk[k];
      if (has_pe) rest += pr[slot == 0 ? RS - 1 : slot - 1];
      const float P = exp2_hw(head + fmaf(cr[slot] - cur_cum, kLog2e, rest));
      if (cval) {
        er[slot] += P;
        da[k] += P;
      }
      sp += P;
    }
    const float St = group_sum<J>(sp);
    // ---- transition gradient: softmax weight of each source label times St ----
    const float invS = 1.0f / S;
#pragma unroll
    for (int r = 0; r < kTRegMax; ++r) {
      const int cs = lj + r * J;
      if (cs < C) tacc[r] += exp2_hw(rw[cs] + tr[cs] - M) * invS * St;
    }
    for (int cs = lj + kTRegMax * J; cs < C; cs += J)
      if (cval) trp[(size_t)cs * C + c] += (double)(exp2_hw(rw[cs] + tr[cs] - M) * invS * St);
    if (cval && lj == 0) {
      q.s_out[((size_t)b * (T + 1) + t) * C + c] = St;
      // row t+1 is complete (all its starts t+1-k >= t0 are done)
      const int r1 = t + 1;
      const int s1 = r1 % RS;
      const float v = er[s1];
      er[s1] = 0.0f;
      if (r1 < t0 + q.TB) e_own_b[(size_t)r1 * C + c] = v;
      else q.halo[(((size_t)b * q.NB + blk) * Kmax + (r1 - t0 - q.TB)) * C + c] = v;
    }
    if (((t - t0) & 63) == 63) flush_acc();
  }
  flush_acc();
  // ---- pending end rows (t1+1 .. t1-1+Kmax), same lane that accumulated them ----
  if (cval && lj == 0) {
    for (int r1 = t1 + 1; r1 <= t1 - 1 + Kmax && r1 <= len; ++r1) {
      const float v = er[r1 % RS];
      if (r1 < t0 + q.TB) e_own_b[(size_t)r1 * C + c] = v;
      else q.halo[(((size_t)b * q.NB + blk) * Kmax + (r1 - t0 - q.TB)) * C + c] = v;
    }
  }
}

// grad_cum / proj grads from the end and start sums, scaled by grad_output.
// Per-block scale of the separate marginals.  Every position lies in exactly one
// segment, so the marginals of the segments covering one position sum to 1.
// Rounding in the fp32 per-step results of the long alpha / beta level chains
// leaves the marginals off by a slowly varying factor; block nb >= 1 measures it
// at t_ref = nb*TB - 1 from the stored alpha and beta tables (every segment
// [s, s+k) with t_ref - Kmax < s <= t_ref < s+k <= len, all labels) and the
// finalize divides the block's sums by it.  Block 0 uses position 0, covered by
// the segments starting there (its start sums).  A value far from 1 (not a
// rounding drift) leaves the block alone (scale 1).  Static transitions, log
// semiring only (the launcher decides).
__global__ void __launch_bounds__(1024) block_coverage_kernel(MargParams q, double* bscale) {
  __shared__ double red[1024 / 64];
  const int b = blockIdx.y, nb = blockIdx.x;
  const int C = q.C, T = q.T, K = q.K, Kmax = q.Kmax;
  const int len = mlen(q.lengths, b, T);
  double acc = 0.0;
  const bool live = len > 0 && nb * q.TB < len;
  if (live && nb == 0) {
    for (int c = threadIdx.x; c < C; c += blockDim.x) acc += (double)q.s_out[(size_t)b * (T + 1) * C + c];
  } else if (live) {
    const int t_ref = nb * q.TB - 1;
    const int s0 = max(0, t_ref - Kmax + 1);
    const size_t row0 = (size_t)b * (T + 1);
    const bool emit = q.emit != nullptr;
    const float* cum_b = emit ? nullptr : q.cum + row0 * C;
    const float* em_b = emit ? q.emit + (size_t)b * T * C : nullptr;
    const int n = (t_ref - s0 + 1) * C;
    for (int w = threadIdx.x; w < n; w += blockDim.x) {
      const int s = s0 + w / C, c = w % C;
      // emission input: cum[e] - cum[s] as a running sum of score rows, from
      // e = t_ref + 1 (rows s .. t_ref) upward
      double dse = 0.0;
      if (emit)
        for (int u = s; u <= t_ref; ++u) dse += (double)em_b[(size_t)u * C + c];
      // forward side: alpha level + u[s,c] (+ proj_start) - cum[s,c] log2 e - log2 Z
      const float* ah = q.aval + (row0 + s) * C;
      float mu = kMinusInf;
      for (int cp = 0; cp < C; ++cp) mu = fmax2(mu, ah[cp] + q.trans[(size_t)cp * C + c] * kLog2e);
      float su = 0.0f;
      for (int cp = 0; cp < C; ++cp) su += exp2_hw((ah[cp] + q.trans[(size_t)cp * C + c] * kLog2e) - mu);
      float ua = mu + log2_hw(su);
      if (q.ps != nullptr) ua += q.ps[((size_t)b * T + s) * C + c] * kLog2e;
      const double A = (q.alvl[row0 + s] + (double)ua) - (emit ? 0.0 : (double)cum_b[(size_t)s * C + c] * kLog2eM) - q.z2[b];
      const int k0 = t_ref - s + 1, k1 = min(Kmax, len - s);
      float sk = 0.0f;
      for (int k = k0; k <= k1; ++k) {
        const int e = s + k;
        float xb = q.bval[(row0 + e) * C + c];
        if (q.pe != nullptr) xb += q.pe[((size_t)b * T + e - 1) * C + c] * kLog2e;
        double x = q.blvl[row0 + e] + (double)xb;
        if (emit) {
          x += dse * kLog2eM;
          dse += (double)em_b[(size_t)min(e, T - 1) * C + c];
        } else {
          x += (double)cum_b[(size_t)e * C + c] * kLog2eM;
        }
        const float dk = q.db[(size_t)(K == 1 ? 0 : min(k, K - 1)) * C + c] * kLog2e;
        sk += exp2_hw((float)(A + x) + dk);
      }
      acc += (double)sk;
    }
  }
  for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    double cov = 0.0;
    for (int i = 0; i < (int)(blockDim.x >> 6); ++i) cov += red[i];
    bscale[(size_t)b * q.NB + nb] = (live && cov > 0.5 && cov < 2.0) ? 1.0 / cov : 1.0;
  }
}

__global__ void finalize_rows_kernel(FinalParams f) {
  const int b = blockIdx.y;
  const int C = f.C, T = f.T;
  const int len = mlen(f.lengths, b, T);
  const float g = f.grad_output[b];
  const size_t n = (size_t)(T + 1) * C;
  // entry (t, c) with its own-row end sum eo and start sum so (loaded by the caller;
  // every row t <= T of the tables exists)
  auto row = [&](int t, int c, size_t o, float eo, float so) {
    float E = 0.0f, S = 0.0f;
    if (t <= len) {
      const int blk = t / f.TB, t0 = blk * f.TB;
      // block scales (coverage pass), 1 without it
      const float ks = (f.bscale != nullptr && blk < f.NB) ? (float)f.bscale[(size_t)b * f.NB + blk] : 1.0f;
      if (t > 0) {
        // own part: written by block blk (absent when t == NB*TB, i.e. t == T)
        if (blk < f.NB) E = ks * eo;
        if (blk >= 1 && t - t0 < f.Kmax) {
          const float kp = f.bscale != nullptr ? (float)f.bscale[(size_t)b * f.NB + blk - 1] : 1.0f;
          E += kp * f.halo[(((size_t)b * f.NB + blk - 1) * f.Kmax + (t - t0)) * C + c];
        }
      }
      if (t < len) S = ks * so;
    }
    if (!f.shift) f.grad_cum[o] = g * (E - S);
    else if (t >= 1) f.grad_cum[((size_t)b * T + t - 1) * C + c] = g * (E - S);
    if (f.grad_ps != nullptr && t < T) f.grad_ps[((size_t)b * T + t) * C + c] = g * S;
    if (f.grad_pe != nullptr && t >= 1) f.grad_pe[((size_t)b * T + t - 1) * C + c] = g * E;
  };
  // four entries per thread loaded before any is used
  const size_t stride = (size_t)gridDim.x * blockDim.x;
  size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (; idx + 3 * stride < n; idx += 4 * stride) {
    int t[4], c[4];
    size_t o[4];
    float eo[4], so[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const size_t id = idx + u * stride;
      t[u] = (int)(id / C);
      c[u] = (int)(id % C);
      o[u] = ((size_t)b * (T + 1) + t[u]) * C + c[u];
      eo[u] = f.e_own[o[u]];
      so[u] = f.s_out[o[u]];
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) row(t[u], c[u], o[u], eo[u], so[u]);
  }
  for (; idx < n; idx += stride) {
    const int t = (int)(idx / C), c = (int)(idx % C);
    const size_t o = ((size_t)b * (T + 1) + t) * C + c;
    row(t, c, o, f.e_own[o], f.s_out[o]);
  }
}

// Shared gradients: sum over sequences (weighted by grad_output) and blocks, in fp64.
// With duration-dependent transitions grad_tr is (trows, C, C): matrix k gets the
// partials of duration k (1 <= k <= Kmax), the others are zero.  One wavefront
// per output element: lane l takes the (sequence, block) partials l, l+64, ...
// and the wave sums them in a fixed order (deterministic).
__global__ void __launch_bounds__(256) finalize_shared_kernel(FinalParams f) {
  const int C = f.C, K = f.K, Kmax = f.Kmax;
  const int n_tr = (f.trows > 0 ? f.trows : 1) * C * C, n_db = K * C;
  const int idx = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (idx >= n_tr + n_db) return;
  const int nparts = f.B * f.NB;
  const double* src = nullptr;
  size_t per = 0, off = 0;
  if (idx < n_tr) {
    const int k = idx / (C * C), e = idx % (C * C);
    if (f.trows == 0 || (k >= 1 && k <= Kmax)) {
      per = (size_t)(f.trows > 0 ? Kmax : 1) * C * C;
      off = (f.trows > 0) ? (size_t)(k - 1) * C * C + e : (size_t)e;
      src = f.tr_part;
    }
  } else {
    const int e = idx - n_tr;
    const int k = e / C, c = e % C;
    // durations mapping to duration-bias row k: k itself (K >= 2, k >= 1) or 1 (K == 1)
    const int dur = (K == 1) ? 1 : k;
    if (dur >= 1 && dur <= Kmax) {
      per = (size_t)Kmax * C;
      off = (size_t)(dur - 1) * C + c;
      src = f.db_part;
    }
  }
  auto term = [&](int j) {
    return (double)f.grad_output[j / f.NB] * (f.bscale != nullptr ? f.bscale[j] : 1.0) * src[(size_t)j * per + off];
  };
  double acc = 0.0;
  if (src != nullptr) {
    // eight partials loaded at once, added in the same order as one at a time
    int j = lane;
    for (; j + 7 * 64 < nparts; j += 8 * 64) {
      double v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = term(j + u * 64);
#pragma unroll
      for (int u = 0; u < 8; ++u) acc += v[u];
    }
    for (; j < nparts; j += 64) acc += term(j);
  }
  for (int m = 32; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
  if (lane == 0) {
    if (idx < n_tr) f.grad_tr[idx] = (float)acc;
    else f.grad_db[idx - n_tr] = (float)acc;
  }
}

// Raw (natural-log) ring checkpoints in the reference's layout, rebuilt from
// the normalised alpha table: ring slot s at checkpoint n holds alpha at the
// position p in (nS-K, nS] with p % K == s (streaming/pytorch_reference.py:192-258).
__global__ void checkpoints_kernel(const float* aval, const double* alvl, const int64_t* lengths, int B, int T,
                                   int C, int K, int S, int n_ckpt, float* out) {
  const size_t total = (size_t)B * n_ckpt * K * C;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (size_t)gridDim.x * blockDim.x) {
    const int c = (int)(idx % C);
    const int s = (int)((idx / C) % K);
    const int n = (int)((idx / ((size_t)C * K)) % n_ckpt);
    const int b = (int)(idx / ((size_t)C * K * n_ckpt));
    const int len = mlen(lengths, b, T);
    const int tn = n * S;
    float v = kNegInf;
    if (tn <= len || n == 0) {
      const int pos = tn - ((tn - s) % K + K) % K;
      if (pos >= 0 && pos <= len) {
        const size_t o = (size_t)b * (T + 1) + pos;
        v = (float)(((double)aval[o * C + c] + alvl[o]) * kLn2);
      }
    }
    out[idx] = v;
  }
}

template <int J>
int launch_marg_j(const Plan& pl, const MargParams& q, hipStream_t st) {
  auto k = marginal_kernel<J>;
  hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl.marg_lds);
  if (e != hipSuccess) return e;
  {
    TimedLaunch tl(kKMarginal, st);
    hipLaunchKernelGGL(k, dim3(pl.B * pl.NB * pl.NCB), dim3(pl.NTM), pl.marg_lds, st, q);
  }
  return hipGetLastError();
}

// Marginals of unit-duration segments (Kmax = 1: K = 1 or 2, the HMM).  Every
// start t has the one segment [t, t+1), so the marginals need no walk over the
// block: P(t,c) = 2^(A[t,c] + x[t+1,c] + db[c]) with
//   A = alpha level + u[t,c] (+ proj_start) - cum[t,c] - log2 Z,
//   x = beta level + beta-hat[t+1,c] (+ proj_end[t]) + cum[t+1,c]
// (cum[t+1]-cum[t] = scores[t] with emission input), and every (t, c) is
// independent.  Thread (lane, c) takes label c of the positions t0+lane,
// t0+lane+NL, ... (NL = 256 / C lanes); its transition-gradient column G[:, c]
// and duration sum accumulate in fp64 registers, then the lanes are summed in
// fp64 through LDS.  The register-
// resident kernel walks a block one position per step (latency-bound: 0.21 ms
// at B=32, T=10^4, C=8).  Outputs: the blocked layout of the other marginal
// kernels (e_own / halo / s_out rows, fp64 block partials).  C <= kUnitMaxC.
constexpr int kUnitMaxC = 16;

__global__ void __launch_bounds__(256) unit_marginal_kernel(MargParams q) {
  extern __shared__ double usm[];  // [NL][C] duration sums, then [NL][C][C] transition sums
  const int C = q.C, T = q.T, K = q.K;
  const int blk = blockIdx.x, b = blockIdx.y;
  const int NL = 256 / C;
  const int tid = threadIdx.x, c = tid % C, lane = tid / C;
  const bool act = lane < NL;
  const int len = mlen(q.lengths, b, T);
  const int t0 = blk * q.TB, own_hi = t0 + q.TB;
  const int t1 = min(own_hi, len);
  const size_t row0 = (size_t)b * (T + 1);
  float* e_own_b = q.e_own + row0 * C;
  float* s_out_b = q.s_out + row0 * C;
  float* halo_b = q.halo + ((size_t)b * q.NB + blk) * C;  // Kmax = 1: one row
  double* dbp = q.db_part + ((size_t)b * q.NB + blk) * C;
  double* trp = q.tr_part + ((size_t)b * q.NB + blk) * C * C;
  const bool emit = q.emit != nullptr;
  double G[kUnitMaxC];
  float trc[kUnitMaxC];
#pragma unroll
  for (int i = 0; i < kUnitMaxC; ++i) {
    G[i] = 0.0;
    trc[i] = (i < C) ? q.trans[(size_t)i * C + c] * kLog2e : 0.0f;  // source i -> destination c
  }
  double D = 0.0;
  const float dbk = q.db[(size_t)(K == 1 ? 0 : 1) * C + c] * kLog2e;  // duration 1: row min(1, K-1)
  const double z2 = q.z2[b];
  if (act && t0 == len && lane == 0) e_own_b[(size_t)len * C + c] = 0.0f;
  if (act && t0 < len) {
    if (lane == 0) e_own_b[(size_t)t0 * C + c] = 0.0f;  // no start of this block ends at t0
    // a position's operands, loaded one iteration ahead (each iteration would otherwise
    // wait for its own loads)
    struct Ops {
      float ah[kUnitMaxC];
      float xb, ps, cu0, cu1;
      double al, bl;
    };
    auto load = [&](int t, Ops& o) {
      const float* ah = q.aval + (row0 + t) * C;
#pragma unroll
      for (int i = 0; i < kUnitMaxC; ++i) o.ah[i] = (i < C) ? ah[i] : 0.0f;
      o.xb = q.bval[(row0 + t + 1) * C + c];
      o.ps = (q.ps != nullptr) ? q.ps[((size_t)b * T + t) * C + c] : 0.0f;
      if (q.pe != nullptr) o.xb += q.pe[((size_t)b * T + t) * C + c] * kLog2e;
      if (emit) {
        o.cu0 = 0.0f;
        o.cu1 = q.emit[((size_t)b * T + t) * C + c];
      } else {
        o.cu0 = q.cum[(row0 + t) * C + c];
        o.cu1 = q.cum[(row0 + t + 1) * C + c];
      }
      o.al = q.alvl[row0 + t];
      o.bl = q.blvl[row0 + t + 1];
    };
    Ops nx;
    if (t0 + lane < t1) load(t0 + lane, nx);
    for (int t = t0 + lane; t < t1; t += NL) {
      const Ops o = nx;
      if (t + NL < t1) load(t + NL, nx);
      const float* ah = o.ah;
      float mx = kMinusInf;
#pragma unroll
      for (int i = 0; i < kUnitMaxC; ++i)
        if (i < C) mx = fmax2(mx, ah[i] + trc[i]);
      float sw = 0.0f;
#pragma unroll
      for (int i = 0; i < kUnitMaxC; ++i)
        if (i < C) sw += exp2_hw((ah[i] + trc[i]) - mx);
      const float u2 = mx + log2_hw(sw);
      float ua = u2, xb = o.xb;
      if (q.ps != nullptr) ua += o.ps * kLog2e;
      const double dc = emit ? (double)o.cu1 * kLog2eM : ((double)o.cu1 - (double)o.cu0) * kLog2eM;
      const double ax = ((o.al + (double)ua) + (o.bl + (double)xb)) - z2;
      const float P = exp2_hw((float)(ax + dc) + dbk);
      s_out_b[(size_t)t * C + c] = P;
      if (t + 1 < own_hi) e_own_b[(size_t)(t + 1) * C + c] = P;
      else halo_b[c] = P;
      D += P;
      // the source weights of u: 2^(alpha-hat + tr - u) = 2^(alpha-hat + tr - mx) / sw
      const float wS = P / sw;
#pragma unroll
      for (int i = 0; i < kUnitMaxC; ++i)
        if (i < C) G[i] += (double)(exp2_hw((ah[i] + trc[i]) - mx) * wS);
    }
  }
  // lanes -> block partials (fp64)
  double* dl = usm;
  double* gl = usm + (size_t)NL * C;
  if (act) {
    dl[lane * C + c] = D;
#pragma unroll
    for (int i = 0; i < kUnitMaxC; ++i)
      if (i < C) gl[((size_t)lane * C + c) * C + i] = G[i];
  }
  __syncthreads();
  for (int e = tid; e < C + C * C; e += blockDim.x) {
    double a = 0.0;
    if (e < C) {
      for (int l = 0; l < NL; ++l) a += dl[l * C + e];
      dbp[e] = a;
    } else {
      const int cs = (e - C) / C, cd = (e - C) % C;  // tr_part[c_src][c_dst]
      for (int l = 0; l < NL; ++l) a += gl[((size_t)l * C + cd) * C + cs];
      trp[(size_t)cs * C + cd] = a;
    }
  }
}

}  // namespace

int launch_marginals(const Plan& pl, const MargParams& q, hipStream_t s) {
  if (pl.dense) return launch_dense_marginals(pl, q, s);
  if (pl.mfast && pl.Kmax == 1 && pl.C <= kUnitMaxC && q.trows == 0) {
    TimedLaunch tl(kKMarginal, s);
    const int NL = 256 / pl.C;
    const size_t lds = sizeof(double) * ((size_t)NL * pl.C + (size_t)NL * pl.C * pl.C);
    hipLaunchKernelGGL(unit_marginal_kernel, dim3(q.NB, pl.B), dim3(256), lds, s, q);
    return hipGetLastError();
  }
  if (pl.mfast) return launch_margfast_j16(pl, q, s);
  switch (pl.JM) {
    case 1: return launch_marg_j<1>(pl, q, s);
    case 2: return launch_marg_j<2>(pl, q, s);
    case 4: return launch_marg_j<4>(pl, q, s);
    case 8: return launch_marg_j<8>(pl, q, s);
    case 16: return launch_marg_j<16>(pl, q, s);
    case 32: return launch_marg_j<32>(pl, q, s);
    case 64: return launch_marg_j<64>(pl, q, s);
    default: return (int)hipErrorInvalidValue;
  }
}

int launch_block_coverage(const Plan& pl, const MargParams& q, double* bscale, hipStream_t s) {
  TimedLaunch tl(kKCoverage, s);
  hipLaunchKernelGGL(block_coverage_kernel, dim3(q.NB, pl.B), dim3(1024), 0, s, q, bscale);
  return hipGetLastError();
}

int launch_finalize(const Plan& pl, const FinalParams& f, hipStream_t s) {
  // at least four entries per thread (the kernel loads four at a time)
  int gx = (int)(((size_t)(pl.T + 1) * pl.C + 1023) / 1024);
  if (gx > 4096) gx = 4096;
  {
    TimedLaunch tl(kKFinalizeRows, s);
    hipLaunchKernelGGL(finalize_rows_kernel, dim3(gx, pl.B), dim3(256), 0, s, f);
  }
  const int n = (f.trows > 0 ? f.trows : 1) * pl.C * pl.C + pl.K * pl.C;
  {
    TimedLaunch tl(kKFinalizeShared, s);
    hipLaunchKernelGGL(finalize_shared_kernel, dim3((n + 3) / 4), dim3(256), 0, s, f);
  }
  return hipGetLastError();
}

int launch_checkpoints(const float* aval, const double* alvl, const int64_t* lengths, int B, int T, int C, int K,
                       int S, int n_ckpt, float* out, hipStream_t s) {
  const size_t total = (size_t)B * n_ckpt * K * C;
  int g = (int)((total + 255) / 256);
  if (g > 8192) g = 8192;
  if (g < 1) g = 1;
  {
    TimedLaunch tl(kKCheckpoints, s);
    hipLaunchKernelGGL(checkpoints_kernel, dim3(g), dim3(256), 0, s, aval, alvl, lengths, B, T, C, K, S, n_ckpt, out);
  }
  return hipGetLastError();
}

}  // namespace tsm
