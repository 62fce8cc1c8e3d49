// Chunk body of the scans with duration-dependent transitions (trows, C, C),
// for gfx950.
//
// With a transition per duration the label mix no longer factors out of the
// duration sum (reference streaming/pytorch_reference.py:104-109 indexes
// transition[k]), so every step costs the full K*C^2 terms:
//   forward : alpha[t,c]  = (+)_{k,c'} alpha[t-k,c'] + trans[k][c',c] + seg(t-k,k,c)
//   backward: beta[t,c']  = (+)_{k,c}  trans[k][c',c] + seg(t,k,c) + beta[t+k,c]
// with seg(s,k,c) = cum[s+k,c]-cum[s,c] + db[min(k,K-1),c] (+ps[s,c]) (+pe[s+k-1,c]).
//
// Thread mapping: a group of J lanes serves one label c; lane j takes the
// durations k = 1+j, 1+j+J, ...  For each of its durations a lane runs over the
// other label axis (forward: sources c' of the ring row of position t-k;
// backward: destinations of the per-step row W[k][:] built in a first stage),
// accumulating every (k, label) term in one online log-sum-exp (or max), and
// the J lanes of the label then combine.  States are normalised per position
// (max over labels subtracted, fp64 level kept) and the chunking, speculation
// and verification are those of the other scans (tsm_chunk_driver.hpp): the
// ring of a chunk boundary is the normalised rows of the last Kmax positions.
//
// Rings are position-major, rows of CS = C|1 words (an odd stride keeps the
// rows that the J lanes of a label read at once on different LDS banks).
#pragma once

#include "tsm_chunk_driver.hpp"

namespace tsm {
namespace dense {

using namespace scan_detail;

constexpr float kInvalid = -1e30f;  // ring value / level difference of a position that does not exist

__host__ __device__ inline int row_stride(int C) { return C | 1; }

template <bool LOGSR>
struct TermAcc {
  Lse2Acc l;
  float m = kMinusInf;
  __device__ __forceinline__ void add8(const float (&x)[8], int n) {
    if constexpr (LOGSR) {
      l.add_batch<8>(x, n);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (i < n) m = fmax2(m, x[i]);
    }
  }
  template <int J>
  __device__ __forceinline__ float reduce() const {
    if constexpr (LOGSR) return group_lse2<J>(l.m, l.s);
    else return group_max<J>(m);
  }
};

// (+) over i < n of a[i] + b[i] + q into acc, in register batches of 8.
template <bool LOGSR>
__device__ __forceinline__ void accumulate_row(TermAcc<LOGSR>& acc, const float* a, const float* bv, float q, int n) {
  for (int i0 = 0; i0 < n; i0 += 8) {
    float x[8];
    const int m = min(8, n - i0);
#pragma unroll
    for (int u = 0; u < 8; ++u)
      if (u < m) x[u] = (a[i0 + u] + bv[i0 + u]) + q;
    acc.add8(x, m);
  }
}

template <int J, bool FWD, bool LOGSR, bool TRL>
struct DenseChunk {
  static constexpr bool kFwd = FWD;
  static constexpr bool kLog = LOGSR;
  static constexpr int kMaxThreads = 1024;
  __device__ static double* red(char* smem, const ScanParams& p) {
    return reinterpret_cast<double*>(smem + dense_lds_layout(p.C, p.Kmax, p.RS, TRL ? 1 : 0).red);
  }

  // Chunk j of sequence b.  FWD: mode 0 exact from position 0, 1 speculative
  // from t_lo - W, 2 exact from (init_st, init_lv) at t_lo; steps t_start+1 ..
  // t_hi.  BWD: mode 0 exact from len, 1 speculative from t_hi + W, 2 exact from
  // the state at t_hi; steps t_start-1 .. t_lo.
  __device__ static void run(const ScanParams& p, char* smem, int b, int j, int mode, const float* init_st,
                             const double* init_lv) {
    const int C = p.C, Kmax = p.Kmax, K = p.K, RS = p.RS, T = p.T;
    const int CS = row_stride(C);
    const int len = seq_len(p, b);
    const int item = b * p.P + j;
    const DenseLds L = dense_lds_layout(C, Kmax, RS, TRL ? 1 : 0);
    float* ring = reinterpret_cast<float*>(smem + L.ring);
    float* crng = reinterpret_cast<float*>(smem + L.crng);
    float* prng = reinterpret_cast<float*>(smem + L.prng);
    double* lring = reinterpret_cast<double*>(smem + L.lring);
    float* dbt = reinterpret_cast<float*>(smem + L.dbt);
    float* wk = reinterpret_cast<float*>(smem + L.wk);
    float* dlt = reinterpret_cast<float*>(smem + L.dlt);
    float* wred = reinterpret_cast<float*>(smem + L.wred);
    float* trl = reinterpret_cast<float*>(smem + L.trk);
    const int TS = TRL ? CS : C;  // row stride of the transition table
    const float* trk = TRL ? trl : p.trx;
    const int tid = threadIdx.x, NT = blockDim.x;
    const int g = tid / J, lj = tid % J;
    const bool cval = g < C;
    const int c = cval ? g : C - 1;  // padding groups shadow the last label and never write
    const int nw = (NT + 63) >> 6, wid = tid >> 6;
    const bool has_ps = p.ps != nullptr, has_pe = p.pe != nullptr;
    const float* cum_b = p.cum + (size_t)b * (T + 1) * C;
    const float* ps_b = has_ps ? p.ps + (size_t)b * T * C : nullptr;
    const float* pe_b = has_pe ? p.pe + (size_t)b * T * C : nullptr;
    const bool store = p.val != nullptr;
    const int jl = bwd_last_chunk(p, len);
    const int t_lo = j * p.Lc;
    const int t_hi = FWD ? min(t_lo + p.Lc, len) : ((j == jl) ? len : (j + 1) * p.Lc);
    // projection folded into ring position pos: forward the start projection
    // ps[pos] of a segment starting there, backward the end projection pe[pos-1]
    auto proj_of = [&](int pos, int cc) -> float {
      if (FWD) return (has_ps && pos < T) ? ps_b[(size_t)pos * C + cc] * kLog2e : 0.0f;
      return (has_pe && pos >= 1) ? pe_b[(size_t)(pos - 1) * C + cc] * kLog2e : 0.0f;
    };

    // ---- constants and empty rings ----
    for (int idx = tid; idx < (Kmax + 1) * C; idx += NT) {
      const int k = idx / C, cc = idx % C;
      const int di = k < K - 1 ? k : K - 1;
      dbt[idx] = (k == 0) ? 0.0f : p.db[(size_t)di * C + cc] * kLog2e;
    }
    if constexpr (TRL) {
      for (int idx = tid; idx < Kmax * C * C; idx += NT) {
        const int r = idx / C, i = idx % C;
        trl[(size_t)r * CS + i] = p.trx[idx];
      }
    }
    for (int idx = tid; idx < RS * CS; idx += NT) {
      ring[idx] = kInvalid;
      crng[idx] = 0.0f;
      prng[idx] = 0.0f;
    }
    for (int i = tid; i < RS; i += NT) lring[i] = 0.0;
    __syncthreads();

    const int t_start = FWD ? (mode == 0 ? 0 : (mode == 1 ? t_lo - p.W : t_lo))
                            : (mode == 0 ? len : (mode == 1 ? t_hi + p.W : t_hi));
    if (mode == 0) {
      // alpha[0] = 0 (forward) / beta[len] = 0 (backward), level 0
      const int pos = t_start;
      for (int cc = tid; cc < C; cc += NT) {
        const int a = (pos % RS) * CS + cc;
        ring[a] = 0.0f;
        crng[a] = cum_b[(size_t)pos * C + cc];
        prng[a] = proj_of(pos, cc);
        if (FWD) {
          if (store && j == 0) p.val[((size_t)b * (T + 1)) * C + cc] = 0.0f;
          if (len == 0) p.fin[(size_t)b * C + cc] = 0.0f;
        } else if (store) {
          p.val[((size_t)b * (T + 1) + len) * C + cc] = 0.0f;
        }
      }
      if (tid == 0) {
        if (FWD) {
          if (store && j == 0) p.lvl[(size_t)b * (T + 1)] = 0.0;
          if (len == 0) p.fin_lvl[b] = 0.0;
        } else if (store) {
          p.lvl[(size_t)b * (T + 1) + len] = 0.0;
        }
      }
      for (int k = tid; k <= Kmax; k += NT) dlt[k] = (k == 1) ? 0.0f : kInvalid;
    } else {
      // the Kmax positions behind (forward) / ahead of (backward) t_start
      for (int idx = tid; idx < Kmax * C; idx += NT) {
        const int i = idx / C, cc = idx % C;
        const int pos = FWD ? t_start - i : t_start + i;
        if (pos < 0 || pos > len) continue;  // does not exist (exact restarts near the ends)
        const int a = (pos % RS) * CS + cc;
        ring[a] = (mode == 1) ? 0.0f : init_st[idx];
        crng[a] = cum_b[(size_t)pos * C + cc];
        prng[a] = proj_of(pos, cc);
      }
      for (int i = tid; i < Kmax; i += NT) {
        const int pos = FWD ? t_start - i : t_start + i;
        if (pos >= 0 && pos <= len) lring[pos % RS] = (mode == 1) ? 0.0 : init_lv[i];
      }
      const double l0 = (mode == 1) ? 0.0 : init_lv[0];
      for (int k = tid; k <= Kmax; k += NT)
        dlt[k] = (k < 1) ? kInvalid : ((k == 1 || mode == 1) ? 0.0f : (float)(init_lv[k - 1] - l0));
    }
    double lvl_prev = (mode == 2) ? init_lv[0] : 0.0;
    __syncthreads();

    const int rec_spec = (mode == 1) ? (FWD ? t_lo : t_hi) : -1;
    const int rec_end = FWD ? ((t_hi < len) ? t_hi : -1) : ((j >= 1) ? t_lo : -1);
    for (int t = FWD ? t_start + 1 : t_start - 1; FWD ? t <= t_hi : t >= t_lo; t += FWD ? 1 : -1) {
      const int s0 = t % RS;
      const float cur_cum = cum_b[(size_t)t * C + c];
      TermAcc<LOGSR> acc;
      if constexpr (FWD) {
        // terms of duration k: ring row of position t-k + trans[k][:, c] + seg
        for (int k = 1 + lj; k <= Kmax; k += J) {
          const float dl = dlt[k];
          if (dl < -1e29f) continue;
          int sl = s0 - k;
          if (sl < 0) sl += RS;
          const int a = sl * CS + c;
          const float q = fmaf(cur_cum - crng[a], kLog2e, (dbt[k * C + c] + prng[a]) + dl);
          accumulate_row<LOGSR>(acc, ring + sl * CS, trk + ((size_t)(k - 1) * C + c) * TS, q, C);
        }
      } else {
        // stage 1: W[k][c] = seg(t,k,c) + beta-hat[t+k,c] + level difference
        const float cur_ps = has_ps ? ps_b[(size_t)t * C + c] * kLog2e : 0.0f;
        for (int k = 1 + lj; k <= Kmax; k += J) {
          const float dl = dlt[k];
          float w = kInvalid;
          if (dl > -1e29f) {
            int sl = s0 + k;
            if (sl >= RS) sl -= RS;
            const int a = sl * CS + c;
            w = fmaf(crng[a] - cur_cum, kLog2e, ((dbt[k * C + c] + prng[a]) + cur_ps) + dl) + ring[a];
          }
          if (cval) wk[(k - 1) * CS + c] = w;
        }
        __syncthreads();  // W complete
        // stage 2: trans[k][c, :] + W[k][:]
        for (int k = 1 + lj; k <= Kmax; k += J) {
          if (dlt[k] < -1e29f) continue;
          accumulate_row<LOGSR>(acc, trk + ((size_t)(k - 1) * C + c) * TS, wk + (k - 1) * CS, 0.0f, C);
        }
      }
      float v2 = acc.template reduce<J>();
      if (FWD && has_pe) v2 += pe_b[(size_t)(t - 1) * C + c] * kLog2e;

      // ---- normaliser: max over labels ----
      const float wm = group_max<64>(v2);
      if ((tid & 63) == 0) wred[wid] = wm;
      __syncthreads();  // A
      float mx = wred[0];
      for (int w = 1; w < nw; ++w) mx = fmax2(mx, wred[w]);
      const double lvl_t = lvl_prev + (double)mx;
      const bool owned = FWD ? (j == 0 || t > t_lo) : (t < t_hi || j == jl);
      // Slot s0 held position t -/+ RS, which no duration k <= Kmax < RS of this
      // step reads, so the row can be replaced before the next barrier.
      if (cval && lj == 0) {
        const float vh = v2 - mx;
        const int a = s0 * CS + c;
        ring[a] = vh;
        crng[a] = cur_cum;
        prng[a] = proj_of(t, c);
        if (store && owned) p.val[((size_t)b * (T + 1) + t) * C + c] = vh;
        if (FWD && t == len) p.fin[(size_t)b * C + c] = vh;
      }
      if (tid == 0) {
        if (store && owned) p.lvl[(size_t)b * (T + 1) + t] = lvl_t;
        if (FWD && t == len) p.fin_lvl[b] = lvl_t;
        lring[s0] = lvl_t;
      }
      // level differences of the next step: dlt[k] = lvl[t' -/+ k] - lvl[t]
      // with t' = t +/- 1 (k = 1 is position t itself)
      const int kcap_next = (mode == 0) ? min(Kmax, FWD ? t + 1 : len - t + 1) : Kmax;
      for (int k = tid + 1; k <= Kmax; k += NT) {
        int sl = FWD ? s0 + 1 - k : s0 - 1 + k;
        if (sl < 0) sl += RS;
        if (sl >= RS) sl -= RS;
        dlt[k] = (k > kcap_next) ? kInvalid : ((k == 1) ? 0.0f : (float)(lring[sl] - lvl_t));
      }
      lvl_prev = lvl_t;
      __syncthreads();  // C

      // ---- boundary states for verification: positions t -/+ i, i < Kmax ----
      if (t == rec_spec || t == rec_end) {
        float* st = (t == rec_spec ? p.st_spec : p.st_end) + (size_t)item * Kmax * C;
        double* lv = (t == rec_spec ? p.lv_spec : p.lv_end) + (size_t)item * Kmax;
        for (int idx = tid; idx < Kmax * C; idx += NT) {
          const int i = idx / C, cc = idx % C;
          const int pos = FWD ? t - i : t + i;
          st[idx] = (pos < 0 || pos > len) ? kInvalid : ring[(pos % RS) * CS + cc];
        }
        for (int i = tid; i < Kmax; i += NT) {
          const int pos = FWD ? t - i : t + i;
          lv[i] = (pos < 0 || pos > len) ? 0.0 : lring[pos % RS];
        }
      }
    }
  }
};

template <int J, bool FWD, bool LOGSR>
int launch_dense_jd(const Plan& pl, const ScanParams& p, hipStream_t st) {
  return pl.dtrl ? launch_chunk_dir<DenseChunk<J, FWD, LOGSR, true>>(pl, p, pl.dense_lds, pl.DNT, st)
                 : launch_chunk_dir<DenseChunk<J, FWD, LOGSR, false>>(pl, p, pl.dense_lds, pl.DNT, st);
}

template <bool FWD>
int launch_dense_dir(const Plan& pl, const ScanParams& p, int semiring, hipStream_t st) {
  const bool lg = semiring == kLog;
  switch (pl.DJ) {
    case 4: return lg ? launch_dense_jd<4, FWD, true>(pl, p, st) : launch_dense_jd<4, FWD, false>(pl, p, st);
    case 16: return lg ? launch_dense_jd<16, FWD, true>(pl, p, st) : launch_dense_jd<16, FWD, false>(pl, p, st);
    case 64: return lg ? launch_dense_jd<64, FWD, true>(pl, p, st) : launch_dense_jd<64, FWD, false>(pl, p, st);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace dense
}  // namespace tsm
