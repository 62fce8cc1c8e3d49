// Chunked forward (alpha) and backward (beta) scans of the semi-Markov
// recursion, factorised and normalised, for gfx950.
//
// Recursion (destination-first edges, reference streaming/pytorch_reference.py:86-111,
// 116-273, 276-525):
//   alpha[t,c] = (+)_{k,c'} alpha[t-k,c'] + seg(t-k,k,c) + trans[c',c]
//   beta[t,c'] = (+)_{k,c}  trans[c',c] + seg(t,k,c) + beta[t+k,c]
// where seg(s,k,c) = cum[s+k,c]-cum[s,c] + db[min(k,K-1),c] (+ps[s,c]) (+pe[s+k-1,c]).
// Because seg does not depend on the source label, both sides factor exactly:
//   forward : u[s,c]  = (+)_{c'} alpha[s,c'] + trans[c',c]        (C^2 per position)
//             alpha[t,c] = (+)_k seg(t-k,k,c) + u[t-k,c]          (K*C per position)
//   backward: w[t,c]  = (+)_k seg(t,k,c) + beta[t+k,c]            (K*C per position)
//             beta[t,c'] = (+)_c trans[c',c] + w[t,c]              (C^2 per position)
// (+) is log-sum-exp (log semiring) or max.  Values are carried in log2 units
// and normalised per position (max over labels subtracted, fp64 level kept).
//
// Parallelism: a sequence of length L is cut into chunks of Lc positions, one
// workgroup each.  Chunk j > 0 starts W positions early from a flat state
// ("warm-up"); the recursion forgets its initial state, and a per-sequence
// fixup kernel verifies that the warmed-up state matches the exact state the
// previous chunk produced up to a constant (the chunk's level offset).  If the
// spread exceeds the tolerance the chunk is recomputed exactly, from the
// previous chunk's state, so the result never depends on the warm-up.
//
// Thread mapping: a group of J consecutive lanes serves one label c; lane j
// handles durations k = 1+j, 1+j+J, ...  Rings are laid out [c][slot] so the J
// lanes of a label read consecutive LDS words.

#include <map>
#include <mutex>
#include <tuple>

#include "tsm_device.hpp"
#include "tsm_internal.hpp"
#include "tsm_chunk_driver.hpp"

namespace tsm {
namespace {

using namespace scan_detail;

constexpr float kInvalid = -1e30f;  // level difference of a duration that does not exist

struct Smem {
  double* lring;
  double* red;
  float* urng;
  float* crng;
  float* dbt;
  float* trt;
  float* row;
  float* dlt;
  float* wred;
};

__device__ inline Smem carve_scan_smem(char* base, const ScanParams& p, int item, bool global_rings) {
  const ScanLds L = scan_lds_layout(p.C, p.KP, p.RS, p.RL, global_rings);
  Smem s;
  s.lring = reinterpret_cast<double*>(base + L.lring);
  s.red = reinterpret_cast<double*>(base + L.red);
  if (!global_rings) {
    s.urng = reinterpret_cast<float*>(base + L.urng);
    s.crng = reinterpret_cast<float*>(base + L.crng);
    s.dbt = reinterpret_cast<float*>(base + L.dbt);
  } else {
    float* g = p.gring + (size_t)item * scan_gring_floats(p.C, p.KP, p.RL);
    s.urng = g;
    s.crng = g + (size_t)p.C * p.RL;
    s.dbt = g + 2 * (size_t)p.C * p.RL;
  }
  s.trt = reinterpret_cast<float*>(base + L.trt);
  s.row = reinterpret_cast<float*>(base + L.row);
  s.dlt = reinterpret_cast<float*>(base + L.dlt);
  s.wred = reinterpret_cast<float*>(base + L.wred);
  return s;
}

// Duration bias (log2) transposed to [c][k], k = 0..KP (row min(k, K-1); 0 for
// k = 0 and k > Kmax), the transition (log2) in the layout the label mix reads,
// and zeroed rings (every slot a padded duration may read holds a finite value).
__device__ inline void load_constants(const ScanParams& p, const Smem& s, bool forward) {
  const int C = p.C, Kmax = p.Kmax, K = p.K, KP = p.KP;
  for (int idx = threadIdx.x; idx < C * (KP + 1); idx += blockDim.x) {
    const int c = idx / (KP + 1), k = idx % (KP + 1);
    const int di = k < K - 1 ? k : K - 1;
    s.dbt[idx] = (k == 0 || k > Kmax) ? 0.0f : p.db[(size_t)di * C + c] * kLog2e;
  }
  for (int idx = threadIdx.x; idx < C * C; idx += blockDim.x) {
    const int a = idx / C, bb = idx % C;
    // forward mix: output label a = c_dst, inner bb = c_src -> trans[c_src][c_dst]
    // backward mix: output label a = c_src, inner bb = c_dst -> trans[c_src][c_dst]
    s.trt[idx] = (forward ? p.trans[(size_t)bb * C + a] : p.trans[(size_t)a * C + bb]) * kLog2e;
  }
  for (int idx = threadIdx.x; idx < C * p.RL; idx += blockDim.x) {
    s.urng[idx] = 0.0f;
    s.crng[idx] = 0.0f;
  }
}

// Forward rings store position pos at a = RS-1-(pos % RS) (and a+RS when a < KP),
// so durations k = 1..KP of step t sit at A_t + k with A_t = RS-1-(t % RS).
__device__ __forceinline__ int fwd_slot(int pos, int RS) { return RS - 1 - pos % RS; }
// Backward rings store position pos at a = pos % RS (and a+RS when a < KP), so
// positions t+k of step t sit at (t % RS) + k.
__device__ __forceinline__ int bwd_slot(int pos, int RS) { return pos % RS; }

__device__ __forceinline__ void ring_put(float* ring_c, int a, float v, int RS, int KP) {
  ring_c[a] = v;
  if (a < KP) ring_c[a + RS] = v;
}

template <bool LOGSR>
struct Acc {
  Lse2Acc l;
  float m = kMinusInf;
  template <int N>
  __device__ __forceinline__ void add(const float (&x)[N], int n) {
    if constexpr (LOGSR) {
      l.add_batch<N>(x, n);
    } else {
#pragma unroll
      for (int i = 0; i < N; ++i)
        if (i < n) m = fmax2(m, x[i]);
    }
  }
  template <int J>
  __device__ __forceinline__ float reduce() const {
    if constexpr (LOGSR) return group_lse2<J>(l.m, l.s);
    else return group_max<J>(m);
  }
};

// (+) over the lane's durations k = k_lane + J*r, r < R, of
//   fmaf(sgn*(cum_ring - cur_cum), log2e, (db + dlt[k]) + state_ring)
// combined across the J lanes of the label.  ul / cl / dl point at the lane's
// first term; term r is J*r floats further.  RMAX > 0: all terms in registers
// (two passes: max, then exponentials); RMAX == 0: batches of 8 with an online
// rescale and the duration bias read from LDS (dr).
template <int J, int RMAX, bool LOGSR, bool FWD>
__device__ __forceinline__ float pull(const float* ul, const float* cl, const float* dl, const float* dr,
                                      const float (&dbr)[RMAX > 0 ? RMAX : 1], float cur_cum, int R) {
  if constexpr (RMAX > 0) {
    // all loads first (kept in flight together), then the arithmetic
    float uv[RMAX], cv[RMAX], dv[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      if (r < R) {
        uv[r] = ul[J * r];
        cv[r] = cl[J * r];
        dv[r] = dl[J * r];
      }
    }
    float xs[RMAX];
#pragma unroll
    for (int r = 0; r < RMAX; ++r) {
      if (r < R) {
        const float content = FWD ? (cur_cum - cv[r]) : (cv[r] - cur_cum);
        xs[r] = fmaf(content, kLog2e, (dbr[r] + dv[r]) + uv[r]);
      }
    }
    float m = kMinusInf;
#pragma unroll
    for (int r = 0; r < RMAX; ++r)
      if (r < R) m = fmax2(m, xs[r]);
    if constexpr (LOGSR) {
      float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
      for (int r = 0; r < RMAX; r += 2) {
        if (r < R) s0 += exp2_hw(xs[r] - m);
        if (r + 1 < R) s1 += exp2_hw(xs[r + 1] - m);
      }
      return group_lse2<J>(m, s0 + s1);
    } else {
      return group_max<J>(m);
    }
  } else {
    Acc<LOGSR> acc;
    for (int r0 = 0; r0 < R; r0 += 8) {
      float xs[8];
      const int n = min(8, R - r0);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        if (u < n) {
          const int o = J * (r0 + u);
          const float content = FWD ? (cur_cum - cl[o]) : (cl[o] - cur_cum);
          xs[u] = fmaf(content, kLog2e, (dr[o] + dl[o]) + ul[o]);
        }
      }
      acc.template add<8>(xs, n);
    }
    return acc.template reduce<J>();
  }
}

// Label mix: out = (+)_{i} (row[i] + trt[cls*C + i]) over the lane's inner
// indices i = j, j+J, ... then combined across the J lanes.
template <int J, bool LOGSR>
__device__ __forceinline__ float label_mix(const float* row, const float* trt, int cls, int j, int C,
                                           float shift) {
  float m = kMinusInf;
  for (int i = j; i < C; i += J) m = fmax2(m, row[i] + trt[cls * C + i]);
  if constexpr (LOGSR) {
    float sm = 0.0f;
    if (m != kMinusInf)
      for (int i = j; i < C; i += J) sm += exp2_hw(row[i] + trt[cls * C + i] - m);
    return group_lse2<J>(m, sm) - shift;
  } else {
    return group_max<J>(m) - shift;
  }
}




// ============================================================================
// forward chunk
// mode 0: exact from position 0; mode 1: speculative from t_lo - W;
// mode 2: exact from the state at t_lo given in (init_st, init_lv).
// Owned positions: [0, t_hi] for chunk 0, (t_lo, t_hi] otherwise.
// State ring entry at position s: u-hat[s] (+ proj_start[s]), i.e. everything
// a segment starting at s contributes that does not depend on its length.
// ============================================================================
template <int J, int RMAX, bool LOGSR, bool GR>
__device__ void forward_chunk(const ScanParams& p, char* smem_base, int b, int j, int mode,
                              const float* init_st, const double* init_lv) {
  const int C = p.C, Kmax = p.Kmax, RS = p.RS, T = p.T, KP = p.KP, RL = p.RL, R = p.R;
  const int len = seq_len(p, b);
  const int t_lo = j * p.Lc;
  const int t_hi = min(t_lo + p.Lc, len);
  const int item = b * p.P + j;
  const bool has_ps = p.ps != nullptr, has_pe = p.pe != nullptr;
  Smem s = carve_scan_smem(smem_base, p, item, GR);
  const int tid = threadIdx.x, NT = blockDim.x;
  const int c_raw = tid / J, lj = tid % J;
  const bool cval = c_raw < C;
  const int c = cval ? c_raw : C - 1;
  const int nw = (NT + 63) >> 6, wid = tid >> 6;
  const float* cum_b = p.cum + (size_t)b * (T + 1) * C;
  const float* ps_b = has_ps ? p.ps + (size_t)b * T * C : nullptr;
  const float* pe_b = has_pe ? p.pe + (size_t)b * T * C : nullptr;
  const bool store = p.val != nullptr;
  const int k_lane = 1 + lj;

  load_constants(p, s, true);
  __syncthreads();
  float dbr[RMAX > 0 ? RMAX : 1];
  if constexpr (RMAX > 0) {
#pragma unroll
    for (int r = 0; r < RMAX; ++r) dbr[r] = (r < R) ? s.dbt[c * (KP + 1) + k_lane + J * r] : 0.0f;
  }
  __syncthreads();
  const int t_start = mode == 0 ? 0 : (mode == 1 ? t_lo - p.W : t_lo);
  float* uc = s.urng + c * RL;
  float* cc_ring = s.crng + c * RL;
  // ---- initial ring ----
  if (mode == 0) {
    // alpha-hat[0] = 0 for all labels, level 0; u[0] = mix of a zero row.
    for (int i = tid; i < C; i += NT) s.row[i] = 0.0f;
    if (tid == 0) s.lring[0] = 0.0;
    __syncthreads();
    const float u0 = label_mix<J, LOGSR>(s.row, s.trt, c, lj, C, 0.0f);
    if (cval && lj == 0) {
      const float ps0 = (has_ps && T > 0) ? ps_b[c] * kLog2e : 0.0f;
      ring_put(uc, fwd_slot(0, RS), u0 + ps0, RS, KP);
      ring_put(cc_ring, fwd_slot(0, RS), cum_b[c], RS, KP);
      if (store && j == 0) p.val[((size_t)b * (T + 1)) * C + c] = 0.0f;
      if (len == 0) p.fin[(size_t)b * C + c] = 0.0f;
    }
    if (tid == 0) {
      if (store && j == 0) p.lvl[(size_t)b * (T + 1)] = 0.0;
      if (len == 0) p.fin_lvl[b] = 0.0;
    }
    for (int k = tid; k <= KP; k += NT) s.dlt[k] = (k == 1) ? 0.0f : kInvalid;
  } else {
    // positions t_start - i, i in [0, Kmax)
    __syncthreads();
    for (int idx = tid; idx < Kmax * C; idx += NT) {
      const int i = idx / C, c2 = idx % C;
      const int pos = t_start - i;
      const float v = (mode == 1) ? (has_ps ? ps_b[(size_t)pos * C + c2] * kLog2e : 0.0f)
                                  : init_st[(size_t)i * C + c2];
      ring_put(s.urng + c2 * RL, fwd_slot(pos, RS), v, RS, KP);
      ring_put(s.crng + c2 * RL, fwd_slot(pos, RS), cum_b[(size_t)pos * C + c2], RS, KP);
    }
    for (int i = tid; i < Kmax; i += NT) s.lring[(t_start - i) % RS] = (mode == 1) ? 0.0 : init_lv[i];
    const double l0 = (mode == 1) ? 0.0 : init_lv[0];
    for (int k = tid; k <= KP; k += NT)
      s.dlt[k] = (k < 1 || k > Kmax) ? kInvalid : ((k == 1 || mode == 1) ? 0.0f : (float)(init_lv[k - 1] - l0));
  }
  double lvl_prev = (mode == 2) ? init_lv[0] : 0.0;
  // Per-step global loads are unconditional (clamped rows; absent projections read
  // cum and are scaled by 0) so the compiler waits on each prefetch precisely
  // instead of draining the whole memory pipeline at branch joins.
  const float* ps_src = has_ps ? ps_b : cum_b;
  const float* pe_src = has_pe ? pe_b : cum_b;
  const float ps_scale = has_ps ? kLog2e : 0.0f;
  const float pe_scale = has_pe ? kLog2e : 0.0f;
  float cur_cum = cum_b[(size_t)min(t_start + 1, T) * C + c];
  float cur_pe = pe_src[(size_t)min(t_start, T - 1) * C + c] * pe_scale;
  __syncthreads();

  const int rec_spec = (mode == 1) ? t_lo : -1;
  for (int t = t_start + 1; t <= t_hi; ++t) {
    // prefetch next-step operands
    const float nxt_cum = cum_b[(size_t)min(t + 1, T) * C + c];
    const float nxt_pe = pe_src[(size_t)min(t, T - 1) * C + c] * pe_scale;
    const float cur_ps = ps_src[(size_t)min(t, T - 1) * C + c] * ps_scale;
    const int A = fwd_slot(t, RS);

    // ---- pull over durations: alpha'[t,c] = (+)_k seg(t-k,k,c) + u[t-k,c] ----
    float a2 = pull<J, RMAX, LOGSR, true>(uc + A + k_lane, cc_ring + A + k_lane, s.dlt + k_lane,
                                          s.dbt + c * (KP + 1) + k_lane, dbr, cur_cum, R);
    a2 += cur_pe;

    // ---- normaliser: max over labels ----
    const float wm = group_max<64>(a2);
    if ((tid & 63) == 0) s.wred[wid] = wm;
    if (cval && lj == 0) s.row[c] = a2;
    __syncthreads();  // A
    float mx = s.wred[0];
    for (int w = 1; w < nw; ++w) mx = fmax2(mx, s.wred[w]);
    const double lvl_t = lvl_prev + (double)mx;
    const bool owned = (j == 0) ? true : (t > t_lo);
    if (cval && lj == 0) {
      const float ah = a2 - mx;
      if (store && owned) p.val[((size_t)b * (T + 1) + t) * C + c] = ah;
      if (t == len) p.fin[(size_t)b * C + c] = ah;
    }
    if (tid == 0) {
      if (store && owned) p.lvl[(size_t)b * (T + 1) + t] = lvl_t;
      if (t == len) p.fin_lvl[b] = lvl_t;
    }
    // level differences for step t+1: dlt[k] = lvl[t+1-k] - lvl[t]
    const int kcap_next = (mode == 0) ? min(Kmax, t + 1) : Kmax;
    for (int k = tid + 1; k <= KP; k += NT)
      s.dlt[k] = (k > kcap_next) ? kInvalid
                                 : ((k == 1) ? 0.0f : (float)(s.lring[wrap_slot(t % RS + 1 - k, RS)] - lvl_t));
    // ---- label mix: u[t,c] = (+)_{c'} alpha-hat[t,c'] + trans[c',c] ----
    const float u2 = label_mix<J, LOGSR>(s.row, s.trt, c, lj, C, mx);
    if (cval && lj == 0) {
      ring_put(uc, A, u2 + cur_ps, RS, KP);
      ring_put(cc_ring, A, cur_cum, RS, KP);
    }
    if (tid == 0) s.lring[t % RS] = lvl_t;
    lvl_prev = lvl_t;
    cur_cum = nxt_cum;
    cur_pe = nxt_pe;
    __syncthreads();  // C
    // ---- boundary states for verification: ring positions t-i, i < Kmax ----
    const bool rec_end = (t == t_hi) && (t_hi < len);
    if (t == rec_spec || rec_end) {
      float* st = (t == rec_spec ? p.st_spec : p.st_end) + (size_t)item * Kmax * C;
      double* lv = (t == rec_spec ? p.lv_spec : p.lv_end) + (size_t)item * Kmax;
      for (int idx = tid; idx < Kmax * C; idx += NT) {
        const int i = idx / C, c2 = idx % C;
        st[idx] = s.urng[c2 * RL + A + i];
      }
      for (int i = tid; i < Kmax; i += NT) lv[i] = s.lring[wrap_slot(t % RS - i, RS)];
    }
  }
}

// ============================================================================
// backward chunk (beta)
// mode 0: exact from position len; mode 1: speculative from t_hi + W;
// mode 2: exact from the state at t_hi given in (init_st, init_lv).
// Owned positions: [t_lo, t_hi) plus len for the last chunk.
// State ring entry at position e: beta-hat[e] (+ proj_end[e-1]), i.e. everything
// a segment ending at e contributes that does not depend on its length.
// ============================================================================
template <int J, int RMAX, bool LOGSR, bool GR>
__device__ void backward_chunk(const ScanParams& p, char* smem_base, int b, int j, int mode,
                               const float* init_st, const double* init_lv) {
  const int C = p.C, Kmax = p.Kmax, RS = p.RS, T = p.T, KP = p.KP, RL = p.RL, R = p.R;
  const int len = seq_len(p, b);
  const int t_lo = j * p.Lc;
  const int jl = bwd_last_chunk(p, len);
  const int t_hi = (j == jl) ? len : (j + 1) * p.Lc;
  const int item = b * p.P + j;
  const bool has_ps = p.ps != nullptr, has_pe = p.pe != nullptr;
  Smem s = carve_scan_smem(smem_base, p, item, GR);
  const int tid = threadIdx.x, NT = blockDim.x;
  const int c_raw = tid / J, lj = tid % J;
  const bool cval = c_raw < C;
  const int c = cval ? c_raw : C - 1;
  const int nw = (NT + 63) >> 6, wid = tid >> 6;
  const float* cum_b = p.cum + (size_t)b * (T + 1) * C;
  const float* ps_b = has_ps ? p.ps + (size_t)b * T * C : nullptr;
  const float* pe_b = has_pe ? p.pe + (size_t)b * T * C : nullptr;
  const bool store = p.val != nullptr;
  const int k_lane = 1 + lj;

  load_constants(p, s, false);
  __syncthreads();
  float dbr[RMAX > 0 ? RMAX : 1];
  if constexpr (RMAX > 0) {
#pragma unroll
    for (int r = 0; r < RMAX; ++r) dbr[r] = (r < R) ? s.dbt[c * (KP + 1) + k_lane + J * r] : 0.0f;
  }
  __syncthreads();
  const int t_start = mode == 0 ? len : (mode == 1 ? t_hi + p.W : t_hi);
  float* uc = s.urng + c * RL;
  float* cc_ring = s.crng + c * RL;
  if (mode == 0) {
    if (cval && lj == 0) {
      const float pe0 = (has_pe && len >= 1) ? pe_b[(size_t)(len - 1) * C + c] * kLog2e : 0.0f;
      ring_put(uc, bwd_slot(len, RS), pe0, RS, KP);
      ring_put(cc_ring, bwd_slot(len, RS), cum_b[(size_t)len * C + c], RS, KP);
      if (store) p.val[((size_t)b * (T + 1) + len) * C + c] = 0.0f;
    }
    if (tid == 0) {
      s.lring[len % RS] = 0.0;
      if (store) p.lvl[(size_t)b * (T + 1) + len] = 0.0;
    }
    for (int k = tid; k <= KP; k += NT) s.dlt[k] = (k == 1) ? 0.0f : kInvalid;
  } else {
    __syncthreads();
    for (int idx = tid; idx < Kmax * C; idx += NT) {
      const int i = idx / C, c2 = idx % C;
      const int pos = t_start + i;
      const float v = (mode == 1) ? (has_pe ? pe_b[(size_t)(pos - 1) * C + c2] * kLog2e : 0.0f)
                                  : init_st[(size_t)i * C + c2];
      ring_put(s.urng + c2 * RL, bwd_slot(pos, RS), v, RS, KP);
      ring_put(s.crng + c2 * RL, bwd_slot(pos, RS), cum_b[(size_t)pos * C + c2], RS, KP);
    }
    for (int i = tid; i < Kmax; i += NT) s.lring[(t_start + i) % RS] = (mode == 1) ? 0.0 : init_lv[i];
    const double l0 = (mode == 1) ? 0.0 : init_lv[0];
    // dlt[k] = lvl[t_start - 1 + k] - lvl[t_start]
    for (int k = tid; k <= KP; k += NT)
      s.dlt[k] = (k < 1 || k > Kmax) ? kInvalid : ((k == 1 || mode == 1) ? 0.0f : (float)(init_lv[k - 1] - l0));
  }
  double lvl_next = (mode == 2) ? init_lv[0] : 0.0;
  // unconditional per-step loads (see forward_chunk)
  const float* ps_src = has_ps ? ps_b : cum_b;
  const float* pe_src = has_pe ? pe_b : cum_b;
  const float ps_scale = has_ps ? kLog2e : 0.0f;
  const float pe_scale = has_pe ? kLog2e : 0.0f;
  float cur_cum = cum_b[(size_t)max(t_start - 1, 0) * C + c];
  __syncthreads();

  const int rec_spec = (mode == 1) ? t_hi : -1;
  const int rec_end = (j >= 1) ? t_lo : -1;
  for (int t = t_start - 1; t >= t_lo; --t) {
    const float nxt_cum = cum_b[(size_t)max(t - 1, 0) * C + c];
    // proj_end of the segment ending at t-1 (folded into ring position t); none for t = 0
    const float pe_prev = pe_src[(size_t)max(t - 1, 0) * C + c] * (t >= 1 ? pe_scale : 0.0f);
    const float cur_ps = ps_src[(size_t)t * C + c] * ps_scale;
    const int A = bwd_slot(t, RS);

    // ---- pull: w[t,c] = (+)_k seg(t,k,c) + beta[t+k,c] ----
    float w2 = pull<J, RMAX, LOGSR, false>(uc + A + k_lane, cc_ring + A + k_lane, s.dlt + k_lane,
                                           s.dbt + c * (KP + 1) + k_lane, dbr, cur_cum, R);
    w2 += cur_ps;

    const float wm = group_max<64>(w2);
    if ((tid & 63) == 0) s.wred[wid] = wm;
    if (cval && lj == 0) s.row[c] = w2;
    __syncthreads();  // A
    float mx = s.wred[0];
    for (int w = 1; w < nw; ++w) mx = fmax2(mx, s.wred[w]);
    const double lvl_t = lvl_next + (double)mx;
    // ---- label mix: beta[t,c'] = (+)_c trans[c',c] + w[t,c] ----
    const float b2 = label_mix<J, LOGSR>(s.row, s.trt, c, lj, C, mx);
    const bool owned = t < t_hi || (j == jl);
    if (cval && lj == 0) {
      if (store && owned) p.val[((size_t)b * (T + 1) + t) * C + c] = b2;
      ring_put(uc, A, b2 + pe_prev, RS, KP);
      ring_put(cc_ring, A, cur_cum, RS, KP);
    }
    if (tid == 0) {
      if (store && owned) p.lvl[(size_t)b * (T + 1) + t] = lvl_t;
      s.lring[A] = lvl_t;
    }
    // dlt for step t-1: lvl[t-1+k] - lvl[t]
    const int kcap_next = (mode == 0) ? min(Kmax, len - t + 1) : Kmax;
    for (int k = tid + 1; k <= KP; k += NT) {
      int slot = A - 1 + k;
      if (slot >= RS) slot -= RS;
      s.dlt[k] = (k > kcap_next) ? kInvalid : ((k == 1) ? 0.0f : (float)(s.lring[slot] - lvl_t));
    }
    lvl_next = lvl_t;
    cur_cum = nxt_cum;
    __syncthreads();  // C
    if (t == rec_spec || t == rec_end) {
      float* st = (t == rec_spec ? p.st_spec : p.st_end) + (size_t)item * Kmax * C;
      double* lv = (t == rec_spec ? p.lv_spec : p.lv_end) + (size_t)item * Kmax;
      for (int idx = tid; idx < Kmax * C; idx += NT) {
        const int i = idx / C, c2 = idx % C;
        st[idx] = s.urng[c2 * RL + A + i];
      }
      for (int i = tid; i < Kmax; i += NT) {
        int slot = A + i;
        if (slot >= RS) slot -= RS;
        lv[i] = s.lring[slot];
      }
    }
  }
}


// Chunk type of the generic scans for the shared chunk driver (tsm_chunk_driver.hpp).
template <int J, int RMAX, bool LOGSR, bool GR, bool FWD>
struct GenericChunk {
  static constexpr bool kFwd = FWD;
  static constexpr bool kLog = LOGSR;
  static constexpr int kMaxThreads = 512;
  __device__ static double* red(char* smem, const ScanParams& p) {
    return reinterpret_cast<double*>(smem + scan_lds_layout(p.C, p.KP, p.RS, p.RL, GR).red);
  }
  __device__ static void run(const ScanParams& p, char* smem, int b, int j, int mode, const float* init_st,
                             const double* init_lv) {
    if constexpr (FWD) forward_chunk<J, RMAX, LOGSR, GR>(p, smem, b, j, mode, init_st, init_lv);
    else backward_chunk<J, RMAX, LOGSR, GR>(p, smem, b, j, mode, init_st, init_lv);
  }
};

// Spread of (exact - speculative) over the boundary state of every speculative
// chunk, all boundaries in parallel: vstat[item] = (max, min) of
//   D[i,c] = (lv_exact[i] - lv_spec[i]) + (st_exact[i,c] - st_spec[i,c])   (fp64)
// where "exact" is the neighbouring chunk's end state (forward: chunk j-1,
// backward: chunk j+1).  Entries unreachable in both (< -1e8 in log2 units) are
// skipped: they add exactly nothing to any later sum.
__global__ void __launch_bounds__(256) verify_kernel(ScanParams p, int forward, int after_retry) {
  __shared__ double red[64];
  if (after_retry) {
    if (*p.vflag == 0) return;  // the retry pass reran nothing: the first verification stands
  } else if (blockIdx.x == 0 && threadIdx.x == 0) {
    *p.vflag = 0;  // the retry pass sets it when it reruns a chunk
  }
  const int b = blockIdx.x / p.P, j = blockIdx.x % p.P;
  const int len = seq_len(p, b);
  const int item = b * p.P + j;
  // chunks that ran speculatively (the status the scan recorded)
  (void)len;
  const bool spec = p.status[item] == 1;
  if (!spec) return;
  const size_t e = forward ? (size_t)(item - 1) : (size_t)(item + 1), sp = (size_t)item;
  double hi, lo;
  boundary_spread_part(p, e, sp, hi, lo);
  double dmax, dmin;
  block_minmax(hi, lo, red, dmax, dmin);
  if (threadIdx.x == 0) {
    p.vstat[2 * sp] = dmax;
    p.vstat[2 * sp + 1] = dmin;
  }
}

// Sequential verification / repair of a sequence's chunks (one block per sequence).
// Add each chunk's frame offset to the levels it owns (global frame afterwards).
__global__ void apply_offsets_kernel(ScanParams p, int forward) {
  const int b = blockIdx.y;
  const int len = seq_len(p, b);
  for (int t = blockIdx.x * blockDim.x + threadIdx.x; t <= len; t += gridDim.x * blockDim.x) {
    int jj;
    if (forward) jj = (t == 0) ? 0 : (t - 1) / p.Lc;
    else jj = min(t / p.Lc, bwd_last_chunk(p, len));
    p.lvl[(size_t)b * (p.T + 1) + t] += p.offs[(size_t)b * p.P + jj];
  }
}

template <int J, int RMAX, bool LOGSR, bool GR>
int launch_dir(const Plan& pl, const ScanParams& p, bool forward, hipStream_t st) {
  return forward ? launch_chunk_dir<GenericChunk<J, RMAX, LOGSR, GR, true>>(pl, p, pl.scan_lds, pl.NT, st)
                 : launch_chunk_dir<GenericChunk<J, RMAX, LOGSR, GR, false>>(pl, p, pl.scan_lds, pl.NT, st);
}

template <int RMAX, bool LOGSR, bool GR>
int launch_j(const Plan& pl, const ScanParams& p, bool fwd, hipStream_t st) {
  switch (pl.J) {
    case 1: return launch_dir<1, RMAX, LOGSR, GR>(pl, p, fwd, st);
    case 2: return launch_dir<2, RMAX, LOGSR, GR>(pl, p, fwd, st);
    case 4: return launch_dir<4, RMAX, LOGSR, GR>(pl, p, fwd, st);
    case 8: return launch_dir<8, RMAX, LOGSR, GR>(pl, p, fwd, st);
    case 16: return launch_dir<16, RMAX, LOGSR, GR>(pl, p, fwd, st);
    case 32: return launch_dir<32, RMAX, LOGSR, GR>(pl, p, fwd, st);
    case 64: return launch_dir<64, RMAX, LOGSR, GR>(pl, p, fwd, st);
    default: return (int)hipErrorInvalidValue;
  }
}

// Instantiated variants: register-resident terms (RMAX = 32) with LDS rings, and
// the generic loop with LDS or workspace rings.
template <bool LOGSR>
int launch_sr(const Plan& pl, const ScanParams& p, bool fwd, hipStream_t st) {
  if (pl.global_rings) return launch_j<0, LOGSR, true>(pl, p, fwd, st);
  // the log semiring's register-resident scan lives in tsm_fastscan.hpp; here
  // only the max semiring keeps a register variant
  if constexpr (!LOGSR) {
    if (pl.RMAX == 32) return launch_j<32, LOGSR, false>(pl, p, fwd, st);
  }
  return launch_j<0, LOGSR, false>(pl, p, fwd, st);
}

int launch_fast(const Plan& pl, const ScanParams& p, bool fwd, hipStream_t st) {
  // the fast path's ring geometry replaces the generic one
  ScanParams q = p;
  q.RS = pl.FRS;
  q.RL = pl.FRL;
  q.R = pl.FR;
  q.KP = pl.FJ * pl.FR;
  switch (pl.FJ) {
    case 8: return launch_fast_j8(pl, q, fwd, st);
    case 16: return launch_fast_j16(pl, q, fwd, st);
    case 32: return launch_fast_j32(pl, q, fwd, st);
    case 64: return launch_fast_j64(pl, q, fwd, st);
    default: return (int)hipErrorInvalidValue;
  }
}

int launch_any(const Plan& pl, const ScanParams& p, int semiring, bool fwd, hipStream_t st) {
  if (pl.dense) {
    // duration-dependent transitions: the dense scan with its own ring geometry
    ScanParams q = p;
    q.RS = pl.DRS;
    return launch_dense_scan(pl, q, semiring, fwd, st);
  }
  if (semiring == kLog && pl.fast) return launch_fast(pl, p, fwd, st);
  if (pl.coop) {
    // the cooperative scan's ring geometry replaces the generic one
    ScanParams q = p;
    q.RS = pl.CRS;
    q.RL = pl.CRL;
    q.R = pl.CR;
    q.KP = 16 * pl.CR;
    return launch_coop_scan(pl, q, fwd, semiring == kLog, st);
  }
  return semiring == kLog ? launch_sr<true>(pl, p, fwd, st) : launch_sr<false>(pl, p, fwd, st);
}

}  // namespace

int launch_scan_viterbi(const Plan& pl, const ScanParams& p, hipStream_t st) {
  ScanParams q = p;
  q.RS = pl.FRS;
  q.RL = pl.FRL;
  q.R = pl.FR;
  q.KP = pl.FJ * pl.FR;
  switch (pl.FJ) {
    case 8: return launch_fast_max_j8(pl, q, st);
    case 16: return launch_fast_max_j16(pl, q, st);
    case 32: return launch_fast_max_j32(pl, q, st);
    case 64: return launch_fast_max_j64(pl, q, st);
    default: return (int)hipErrorInvalidValue;
  }
}

int launch_verify(const Plan& pl, const ScanParams& p, bool forward, hipStream_t st, bool after_retry) {
  if (pl.P > 1) {
    TimedLaunch tl(kKVerify, st);
    hipLaunchKernelGGL(verify_kernel, dim3(pl.B * pl.P), dim3(256), 0, st, p, forward ? 1 : 0, after_retry ? 1 : 0);
  }
  return hipGetLastError();
}

int launch_apply_offsets(const Plan& pl, const ScanParams& p, bool forward, hipStream_t st) {
  if (p.lvl != nullptr) {
    const int per = 256;
    int gx = (pl.T + 1 + per - 1) / per;
    if (gx > 1024) gx = 1024;
    TimedLaunch tl(kKApplyOffsets, st);
    hipLaunchKernelGGL(apply_offsets_kernel, dim3(gx, pl.B), dim3(per), 0, st, p, forward ? 1 : 0);
  }
  return hipGetLastError();
}

int launch_scan_backward_fused(const Plan& pl, const ScanParams& p, hipStream_t st) {
  if (!pl.fast || pl.FJ != 16 || pl.FSB < 4 || pl.fstage == 0) return (int)hipErrorInvalidValue;
  ScanParams q = p;
  q.RS = pl.FRS;
  q.RL = pl.FRL;
  q.SB = pl.FSB;
  q.R = pl.FR;
  q.KP = 16 * pl.FR;
  return pl.FR <= 16 ? launch_fused_j16_lo(pl, q, st) : launch_fused_j16_hi(pl, q, st);
}

int fast_scan_regs(const Plan& pl, int kind) {
  // one query per instance (kind, lanes per label, durations per lane, mix width)
  static std::mutex mu;
  static std::map<std::tuple<int, int, int, int>, int> cache;
  const int cj = (pl.FJ == 8 && pl.FR == 1 && pl.C <= 8) ? 1 : (pl.C <= 2 * pl.FJ ? 2 : 4);
  const auto key = std::make_tuple(kind, pl.FJ, pl.FR, cj);
  {
    std::lock_guard<std::mutex> lk(mu);
    const auto it = cache.find(key);
    if (it != cache.end()) return it->second;
  }
  int regs = -1;
  ScanParams q{};
  q.B = pl.B;
  q.T = pl.T;
  q.C = pl.C;
  q.K = pl.K;
  q.Kmax = pl.Kmax;
  q.query_regs = &regs;
  const int e = kind == 2 ? launch_scan_viterbi(pl, q, nullptr) : launch_fast(pl, q, kind == 0, nullptr);
  if (e != hipSuccess || regs <= 0) return -1;  // not cached: no device yet
  std::lock_guard<std::mutex> lk(mu);
  cache[key] = regs;
  return regs;
}

int launch_scan_forward(const Plan& pl, const ScanParams& p, int semiring, hipStream_t s) {
  return launch_any(pl, p, semiring, true, s);
}
int launch_scan_backward(const Plan& pl, const ScanParams& p, int semiring, hipStream_t s) {
  return launch_any(pl, p, semiring, false, s);
}

}  // namespace tsm
