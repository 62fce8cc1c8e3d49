// Register-resident segment marginals for gfx950 (companion of tsm_fastscan.hpp).
//
// Given the stored forward table (alpha-hat, fp64 levels) and backward table
// (beta-hat, levels), every start position t is independent:
//   P(t,k,c) = exp2( A[t,c] + x[t+k,c] + db[k,c] )
//   A[t,c]   = lvl_a[t] + u[t,c] (+ ps[t,c]) - cum[t,c]*log2(e) - log2 Z
//   x[e,c]   = lvl_b[e] + beta-hat[e,c] (+ pe[e-1,c]) + cum[e,c]*log2(e)
//   u[t,c]   = log2 sum_{c'} 2^(alpha-hat[t,c'] + trans[c',c])
// (all log2 units; the large level and cumulative-score parts cancel in fp64,
// only the final exponent is rounded to fp32).  The gradients need
//   S[t,c] = sum_k P            (start sums: grad_cum[t] -= S, grad_ps[t] += S)
//   E[e,c] = sum_k P(e-k,k,c)   (end sums: grad_cum[e] += E, grad_pe[e-1] += E)
//   D[k,c] = sum_t P            (grad duration_bias)
//   G[c',c] = sum_t S[t,c] * 2^(alpha-hat[t,c'] + trans[c',c] - u[t,c])   (grad trans)
//
// One wavefront serves 4 labels of one position block: a 16-lane group (one
// DPP row) per label, lane j owning durations k = 1 + j + 16*r (r < R, the
// compile-time mapping of the scans).  x lives in a linear LDS ring per label
// (the KP = 16*R terms of a step are contiguous; every few batches the live
// KP entries move to the front), staged 16 positions at a time, together with
// the per-step operands, from loads issued one batch earlier.  The alpha-hat
// row of a step (the label mix's sources) goes straight from global memory to
// registers, loaded one step ahead.  E lives in registers: lane j's register r
// holds the running end sum of position t+1+j+16r, so after each step the
// sums slide one lane down the row (DPP row rotate; lane 0 first takes its
// next register) and position t+1, complete, leaves from lane 0.  D and G
// accumulate in fp32 registers; every 64 steps they are folded into the
// block's fp64 partials in global memory with non-returning atomic adds (each
// lane owns its entries), so no fp64 accumulators hold registers.  The
// duration biases stay fp32 and are added after the fp64 sum x + A, whose
// large parts cancel.  Waves never synchronise with each other.
// Outputs follow the blocked layout of the generic marginal kernel (e_own /
// halo / s_out rows, fp64 per-block partials), so the same finalize kernels
// produce the gradients.
// Emission input (q.emit != null): the kernel reads the projected scores
// (B, T, C) and builds cum itself in fp64, in the block's own frame (cum = 0
// at t0): each batch of J positions of the x stream and of the step stream is
// one 16-lane prefix sum of its score rows plus the stream's running total
// (kept in LDS).  Only differences of cum along one label enter P, so the
// frame drops out.
#pragma once

#include "tsm_device.hpp"
#include "tsm_internal.hpp"

namespace tsm {
namespace margfast {

constexpr double kInvD = -1e30;
constexpr double kLog2eD = 1.4426950408889634;

__device__ __forceinline__ void wave_lds_order() { __asm__ volatile("" ::: "memory"); }

__device__ __forceinline__ int mlen(const int64_t* lengths, int b, int T) {
  int64_t L = lengths[b];
  if (L < 0) L = 0;
  if (L > T) L = T;
  return (int)L;
}

constexpr int kDppRowRor15 = 0x12F;  // row_ror:15 -- lane i reads lane (i+1) mod 16 of its row

// a + (rot of lane (i+1) mod 16 of the row), one v_add_f32 with a DPP source.
// The compiler does not fuse the rotation into the add here (it hoists the DPP
// move away from it), which costs two more instructions per end sum.  The
// s_nop gives the two wait states a DPP read needs after a VALU write, which
// the compiler does not track across inline asm.  All lanes are active.
__device__ __forceinline__ float add_row_ror15(float rot, float a) {
  float r;
  asm("s_nop 1\n\tv_add_f32_dpp %0, %1, %2 row_ror:15 row_mask:0xf bank_mask:0xf bound_ctrl:1"
      : "=v"(r) : "v"(rot), "v"(a));
  return r;
}

// CJ source labels per lane in the label mix (C <= CJ * J).
template <int J, int R, int CJ>
__global__ void __launch_bounds__(64) margfast_kernel(MargParams q) {
  static_assert(J == 16, "end sums slide along one 16-lane DPP row");
  constexpr int kCJ = CJ;
  extern __shared__ __align__(16) char smem[];
  constexpr int KP = J * R;
  constexpr int CB = 64 / J;
  // The NCB label blocks of one position block read the same alpha-hat rows:
  // they take block ids with equal blockIdx % 8, which the dispatcher places on
  // one XCD (one L2), and follow each other there.  The grid is padded to whole
  // groups of 8 position blocks; padding blocks do nothing.
  const int xcd = blockIdx.x & 7, w = blockIdx.x >> 3;
  const int cbk = w % q.NCB;
  const int pb = (w / q.NCB) * 8 + xcd;
  if (pb >= q.B * q.NB) return;
  const int blk = pb % q.NB;
  const int b = pb / q.NB;
  const int C = q.C, Kmax = q.Kmax, K = q.K, T = q.T, RL = q.RL;
  const int lane = threadIdx.x, g = lane / J, lj = lane % J;
  const int c_raw = cbk * CB + g;
  const bool cval = c_raw < C;
  const int c = cval ? c_raw : C - 1;
  const int len = mlen(q.lengths, b, T);
  const int t0 = blk * q.TB;
  float* e_own_b = q.e_own + (size_t)b * (T + 1) * C;
  double* dbp = q.db_part + ((size_t)b * q.NB + blk) * Kmax * C;
  double* trp = q.tr_part + ((size_t)b * q.NB + blk) * C * C;
  if (t0 >= len) {
    // no starts here: zero this block's partials (they are summed over all
    // blocks) and the end sum at len when the block begins there
    if (cval) {
      for (int k = lj; k < Kmax; k += J) dbp[(size_t)k * C + c] = 0.0;
      for (int cs = lj; cs < C; cs += J) trp[(size_t)cs * C + c] = 0.0;
      if (t0 == len && lj == 0) e_own_b[(size_t)len * C + c] = 0.0f;
    }
    return;
  }
  const int t1 = min(t0 + q.TB, len);
  if (cval) {
    for (int k = lj; k < Kmax; k += J) dbp[(size_t)k * C + c] = 0.0;
    for (int cs = lj; cs < C; cs += J) trp[(size_t)cs * C + c] = 0.0;
  }
  __threadfence();  // the zeros before the first atomic add
  const bool has_ps = q.ps != nullptr, has_pe = q.pe != nullptr;
  const bool emit = q.emit != nullptr;
  const float* cum_b = emit ? nullptr : q.cum + (size_t)b * (T + 1) * C;
  const float* em_b = emit ? q.emit + (size_t)b * T * C : nullptr;
  // per position e: cum[e] (cum input) or the score row e-1 stepped over to reach e
  auto xs_at = [&](int e) -> float {
    if (!emit) return cum_b[(size_t)e * C + c];
    const int r = e - 1 < 0 ? 0 : (e - 1 > T - 1 ? T - 1 : e - 1);
    return em_b[(size_t)r * C + c];
  };
  const float* ps_b = has_ps ? q.ps + (size_t)b * T * C : nullptr;
  const float* pe_b = has_pe ? q.pe + (size_t)b * T * C : nullptr;
  const float* av_b = q.aval + (size_t)b * (T + 1) * C;
  const double* al_b = q.alvl + (size_t)b * (T + 1);
  const float* bv_b = q.bval + (size_t)b * (T + 1) * C;
  const double* bl_b = q.blvl + (size_t)b * (T + 1);
  const double z2 = q.z2[b];

  const MargFastLds L = margfast_lds_layout(CB, RL, J, C);
  double* xr = reinterpret_cast<double*>(smem + L.xring) + (size_t)g * RL;
  // per-step operands of the current batch of J positions [tb, tb+J)
  double* alv = reinterpret_cast<double*>(smem + L.alv);  // [J]    alpha levels
  double* cmv = reinterpret_cast<double*>(smem + L.cmv);  // [CB][J] cum of own labels
  double* crr = reinterpret_cast<double*>(smem + L.carry) + 2 * g;  // emission input: x / step stream totals
  float* psv = reinterpret_cast<float*>(smem + L.psv);    // [CB][J] proj_start of own labels

  // ---- constants ----
  float dbr[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int k = 1 + lj + J * r;
    const int di = k < K - 1 ? k : K - 1;
    dbr[r] = (k <= Kmax) ? q.db[(size_t)di * C + c] * kLog2e : (float)kInvD;
  }
  float trr[kCJ];
#pragma unroll
  for (int i = 0; i < kCJ; ++i) {
    const int ci = lj + J * i;
    trr[i] = (ci < C) ? q.trans[(size_t)ci * C + c] * kLog2e : 0.0f;  // source ci -> destination c
  }

  // x of position e (own label), or "does not exist" beyond len
  auto x_of = [&](int e, float bv, double bl, double cm, float pe) -> double {
    return (e <= len) ? (bl + (double)(bv + pe)) + cm * kLog2eD : kInvD;
  };
  // emission input: cum of one batch of J consecutive positions from their score
  // rows d (inclusive prefix over the group) and the stream's total before them
  auto em_scan = [&](float d, double& total) -> double {
    double v = (double)d;
#pragma unroll
    for (int o = 1; o < J; o <<= 1) {
      const double w = __shfl_up(v, o, J);
      if (lj >= o) v += w;
    }
    const double val = total + v;
    total = __shfl(val, J - 1, J);
    return val;
  };
  auto clampT = [&](int e) { return e > T ? T : e; };

  // ---- initial ring: x for positions t0+1 .. t0+KP ----
  // The ring is linear: position p sits at index p - ofs (wave-uniform), each
  // batch appends J positions, and when the next batch would run past RL
  // entries the KP live positions move to the front.
  int ofs = t0 + 1;
  double xtot = 0.0;  // emission input: cum of the x stream's last position (t0: 0)
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const int e = t0 + 1 + lj + J * r;
    const int ec = clampT(e);
    const float pe = (has_pe && ec >= 1) ? pe_b[(size_t)(ec - 1) * C + c] * kLog2e : 0.0f;
    const double cm = emit ? em_scan(xs_at(e), xtot) : (double)xs_at(ec);
    xr[e - ofs] = x_of(e, bv_b[(size_t)ec * C + c], bl_b[ec], cm, pe);
  }
  if (emit && lj == 0) {
    crr[0] = xtot;
    crr[1] = 0.0;  // the step stream starts at t0, cum 0
  }
  // Batches of J steps.  At a batch start tb the registers loaded one batch
  // earlier are written to LDS -- x for positions tb+KP+1 .. tb+KP+J and the
  // operands of steps tb .. tb+J-1 -- and the next batch's loads are issued.
  int e_n = t0 + KP + 1 + lj;  // x position this lane stages at the next batch start
  float sb_bv, sb_cm, sb_pe;
  double sb_bl;
  double ral;
  float rcm, rps;
  auto load_batch = [&](int tb, int e) {
    const int ec = clampT(e);
    sb_bv = bv_b[(size_t)ec * C + c];
    sb_bl = bl_b[ec];
    sb_cm = emit ? xs_at(e) : xs_at(ec);
    sb_pe = (has_pe && ec >= 1) ? pe_b[(size_t)(ec - 1) * C + c] * kLog2e : 0.0f;
    ral = al_b[clampT(tb + (lane % J))];
    const int tp = clampT(tb + lj);
    // emission input: position t0 adds nothing to its stream
    rcm = emit ? (tb + lj > t0 ? xs_at(tb + lj) : 0.0f) : xs_at(tp);
    rps = has_ps ? ps_b[(size_t)min(tp, T - 1) * C + c] : 0.0f;
  };
  load_batch(t0, e_n);
  // alpha-hat row of step tp: this lane's CJ source labels (clamped into the row;
  // the label mix masks the clamped ones)
  float rvn[kCJ];
  auto load_row = [&](int tp) {
    const float* rowp = av_b + (size_t)clampT(tp) * C;
#pragma unroll
    for (int i = 0; i < kCJ; ++i) rvn[i] = rowp[min(lj + J * i, C - 1)];
  };
  load_row(t0);
  if (cval && lj == 0) e_own_b[(size_t)t0 * C + c] = 0.0f;
  wave_lds_order();

  float d32[R];
  float ea[R];  // running end sums of positions t+1+lj+16r (this block's starts)
  const int lane0 = (lj == 0) ? -1 : 0;  // all bits set on the row's lane 0
#pragma unroll
  for (int r = 0; r < R; ++r) {
    d32[r] = 0.0f;
    ea[r] = 0.0f;
  }
  float g32[kCJ];
#pragma unroll
  for (int i = 0; i < kCJ; ++i) g32[i] = 0.0f;
  // D and G partials: fp32 sums since the last fold added into the zeroed fp64
  // block partials.  Addresses and masks come from an opaque copy of the lane
  // index: otherwise they are hoisted out of the step loop into registers.
  auto fold = [&]() {
    int ljo = lj;
    __asm__ volatile("" : "+v"(ljo));
    double* a = dbp + (size_t)ljo * C + c;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      if (cval && 1 + ljo + J * r <= Kmax) unsafeAtomicAdd(a, (double)d32[r]);
      a += (size_t)J * C;
      d32[r] = 0.0f;
    }
    double* tg = trp + (size_t)ljo * C + c;
#pragma unroll
    for (int i = 0; i < kCJ; ++i) {
      if (cval && ljo + J * i < C) unsafeAtomicAdd(tg, (double)g32[i]);
      tg += (size_t)J * C;
      g32[i] = 0.0f;
    }
  };
  float* s_out_b = q.s_out + (size_t)b * (T + 1) * C;
  float* halo_b = q.halo + ((size_t)b * q.NB + blk) * Kmax * C;
  // end rows [t0, own_hi) are this block's own; rows own_hi .. own_hi+Kmax-1 go to the
  // halo that the next block's rows add in the finalize kernel
  const int own_hi = t0 + q.TB;

  for (int t = t0; t < t1; ++t) {
    const int ib = (t - t0) % J;  // step within the batch
    if (ib == 0) {
      if (t + KP + J - ofs >= RL) {  // the batch's last index t+KP+J-ofs must stay below RL
        // positions t+1 .. t+KP to indices 0 .. KP-1, ascending: each lane moves
        // only its own entries, and overwrites only ones it has already moved
        const int sh = t + 1 - ofs;
#pragma unroll
        for (int r = 0; r < R; ++r) xr[lj + J * r] = xr[sh + lj + J * r];
        ofs = t + 1;
        wave_lds_order();
      }
      double cme = (double)sb_cm, cmt = (double)rcm;
      if (emit) {
        double xt = crr[0], st = crr[1];
        cme = em_scan(sb_cm, xt);
        cmt = em_scan(rcm, st);
        wave_lds_order();
        if (lj == 0) {
          crr[0] = xt;
          crr[1] = st;
        }
      }
      xr[e_n - ofs] = x_of(e_n, sb_bv, sb_bl, cme, sb_pe);
      if (lane < J) alv[lane] = ral;
      cmv[g * J + lj] = cmt;
      psv[g * J + lj] = rps;
      e_n += J;
      load_batch(t + J, e_n);
      wave_lds_order();
    }
    // ---- this step's operands ----
    float rv[kCJ];
#pragma unroll
    for (int i = 0; i < kCJ; ++i) rv[i] = rvn[i];
    load_row(t + 1);
    const double al = alv[ib];
    const double cm = cmv[g * J + ib];
    const float ps_t = psv[g * J + ib];
    // ---- u[t,c] and the softmax weights of the source labels ----
    float mq = kMinusInf;
#pragma unroll
    for (int i = 0; i < kCJ; ++i)
      if (lj + J * i < C) mq = fmax2(mq, rv[i] + trr[i]);
    const float M = group_max<J>(mq);
    float ew[kCJ];
    float sw = 0.0f;
#pragma unroll
    for (int i = 0; i < kCJ; ++i) {
      ew[i] = (lj + J * i < C) ? exp2_hw((rv[i] + trr[i]) - M) : 0.0f;
      sw += ew[i];
    }
    const float S = group_sum<J>(sw);
    const float u2 = M + log2_hw(S);
    const double At = ((al + (double)(u2 + ps_t * kLog2e)) - cm * kLog2eD) - z2;

    // ---- segment marginals over the lane's durations ----
    // The previous step's end sums slide to positions t+1+lj+16r: lane 0 takes its
    // next register (dropping the row it flushed), then the row rotates one lane
    // down (lane j takes lane j+1), fused with the accumulation.  Ascending r
    // reads ea[r+1] before it is updated.
    const double* xb = xr + (t + 1 - ofs + lj);
    float sp0 = 0.0f, sp1 = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const float P = exp2_hw((float)(xb[J * r] + At) + dbr[r]);
      d32[r] += P;
      if (r & 1) sp1 += P;
      else sp0 += P;
      // a bitwise merge: a select between ea[r + 1] and ea[r] would be turned
      // into one register-array read at a lane-dependent index
      const float nxt = (r + 1 < R) ? ea[r + 1] : 0.0f;
      const float sl = __int_as_float((__float_as_int(nxt) & lane0) | (__float_as_int(ea[r]) & ~lane0));
      ea[r] = add_row_ror15(sl, P);
    }
    const float St = group_sum<J>(sp0 + sp1);
    // ---- transition gradient: softmax weight of each source label times S[t,c] ----
    const float wS = St / S;
#pragma unroll
    for (int i = 0; i < kCJ; ++i) g32[i] = fmaf(ew[i], wS, g32[i]);
    if (cval && lj == 0) {
      s_out_b[(size_t)t * C + c] = St;
      // end row t+1 is complete (all its starts t+1-k >= t0 are done)
      const int p = t + 1;
      if (p < own_hi) e_own_b[(size_t)p * C + c] = ea[0];
      else halo_b[(size_t)(p - own_hi) * C + c] = ea[0];
    }
    if (((t - t0) & 63) == 63) fold();
  }
  // ---- pending end rows t1+1 .. t1+Kmax-1 (partial sums from this block's starts) ----
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const float nxt = (r + 1 < R) ? ea[r + 1] : 0.0f;
    ea[r] = dpp_f<kDppRowRor15>(__int_as_float((__float_as_int(nxt) & lane0) | (__float_as_int(ea[r]) & ~lane0)));
  }
  if (cval) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int p = t1 + 1 + lj + J * r;
      if (p <= t1 - 1 + Kmax && p <= len) {
        if (p < own_hi) e_own_b[(size_t)p * C + c] = ea[r];
        else halo_b[(size_t)(p - own_hi) * C + c] = ea[r];
      }
    }
  }
  // ---- block partials: the sums since the last fold ----
  fold();
}

template <int J, int R, int CJ = 4>
int launch_margfast_jr(const Plan& pl, const MargParams& q, hipStream_t st) {
  auto k = margfast_kernel<J, R, CJ>;
  hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl.marg_lds);
  if (e != hipSuccess) return e;
  TimedLaunch tl(kKMarginal, st);
  const int npb = (pl.B * pl.NB + 7) / 8 * 8;  // position blocks, padded to groups of 8
  hipLaunchKernelGGL(k, dim3(npb * pl.NCB), dim3(64), pl.marg_lds, st, q);
  return hipGetLastError();
}

}  // namespace margfast
}  // namespace tsm
