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

#include "tsm_device.hpp"
#include "tsm_internal.hpp"

namespace tsm {
namespace {

struct Smem {
  double* lring;
  double* red;
  float* urng;
  float* crng;
  float* prng;
  float* dbt;
  float* trt;
  float* row;
  float* dlt;
  float* wred;
};

__device__ inline Smem carve_scan_smem(char* base, const ScanParams& p, int item, bool has_proj,
                                       bool global_rings) {
  const ScanLds L = scan_lds_layout(p.C, p.Kmax, p.RS, has_proj, global_rings);
  Smem s;
  s.lring = reinterpret_cast<double*>(base + L.lring);
  s.red = reinterpret_cast<double*>(base + L.red);
  if (!global_rings) {
    s.urng = reinterpret_cast<float*>(base + L.urng);
    s.crng = reinterpret_cast<float*>(base + L.crng);
    s.prng = reinterpret_cast<float*>(base + L.prng);
    s.dbt = reinterpret_cast<float*>(base + L.dbt);
  } else {
    float* g = p.gring + (size_t)item * scan_gring_floats(p.C, p.Kmax, p.RS);
    const size_t ring = (size_t)p.C * p.RS;
    s.urng = g;
    s.crng = g + ring;
    s.prng = g + 2 * ring;
    s.dbt = g + 3 * ring;
  }
  s.trt = reinterpret_cast<float*>(base + L.trt);
  s.row = reinterpret_cast<float*>(base + L.row);
  s.dlt = reinterpret_cast<float*>(base + L.dlt);
  s.wred = reinterpret_cast<float*>(base + L.wred);
  return s;
}

// Duration bias (log2) transposed to [c][k], k = 1..Kmax (index min(k, K-1)),
// and the transition (log2) in the layout the label mix reads.
__device__ inline void load_constants(const ScanParams& p, const Smem& s, bool forward) {
  const int C = p.C, Kmax = p.Kmax, K = p.K;
  for (int idx = threadIdx.x; idx < C * (Kmax + 1); idx += blockDim.x) {
    const int c = idx / (Kmax + 1), k = idx % (Kmax + 1);
    const int di = k < K - 1 ? k : K - 1;
    s.dbt[idx] = (k == 0) ? 0.0f : p.db[(size_t)di * C + c] * kLog2e;
  }
  for (int idx = threadIdx.x; idx < C * C; idx += blockDim.x) {
    const int a = idx / C, bb = idx % C;
    // forward mix: output label a = c_dst, inner bb = c_src -> trans[c_src][c_dst]
    // backward mix: output label a = c_src, inner bb = c_dst -> trans[c_src][c_dst]
    s.trt[idx] = (forward ? p.trans[(size_t)bb * C + a] : p.trans[(size_t)a * C + bb]) * kLog2e;
  }
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

__device__ inline int seq_len(const ScanParams& p, int b) {
  int64_t L = p.lengths[b];
  if (L < 0) L = 0;
  if (L > p.T) L = p.T;
  return (int)L;
}

// Backward chunks own [j*Lc, (j+1)*Lc); the last one, jl, also owns position len.
// jl = (len-1)/Lc keeps jl < P even when len is a multiple of Lc.
__device__ inline int bwd_last_chunk(const ScanParams& p, int len) { return len > 0 ? (len - 1) / p.Lc : 0; }

// ============================================================================
// forward chunk
// mode 0: exact from position 0; mode 1: speculative from t_lo - W;
// mode 2: exact from the state at t_lo given in (init_st, init_lv).
// Owned positions: [0, t_hi] for chunk 0, (t_lo, t_hi] otherwise.
// ============================================================================
template <int J, bool LOGSR, bool GR>
__device__ void forward_chunk(const ScanParams& p, char* smem_base, int b, int j, int mode,
                              const float* init_st, const double* init_lv) {
  const int C = p.C, Kmax = p.Kmax, RS = p.RS, T = p.T;
  const int len = seq_len(p, b);
  const int t_lo = j * p.Lc;
  const int t_hi = min(t_lo + p.Lc, len);
  const int item = b * p.P + j;
  const bool has_ps = p.ps != nullptr, has_pe = p.pe != nullptr;
  Smem s = carve_scan_smem(smem_base, p, item, has_ps, GR);
  const int tid = threadIdx.x, NT = blockDim.x;
  const int c_raw = tid / J, lj = tid % J;
  const bool cval = c_raw < C;
  const int c = cval ? c_raw : C - 1;
  const int nw = (NT + 63) >> 6, wid = tid >> 6;
  const float* cum_b = p.cum + (size_t)b * (T + 1) * C;
  const float* ps_b = has_ps ? p.ps + (size_t)b * T * C : nullptr;
  const float* pe_b = has_pe ? p.pe + (size_t)b * T * C : nullptr;
  const bool store = p.val != nullptr;

  load_constants(p, s, true);
  const int t_start = mode == 0 ? 0 : (mode == 1 ? t_lo - p.W : t_lo);
  // ---- initial ring ----
  if (mode == 0) {
    // alpha-hat[0] = 0 for all labels, level 0; u[0] = mix of a zero row.
    for (int i = tid; i < C; i += NT) s.row[i] = 0.0f;
    if (tid == 0) s.lring[0] = 0.0;
    __syncthreads();
    const float u0 = label_mix<J, LOGSR>(s.row, s.trt, c, lj, C, 0.0f);
    if (cval && lj == 0) {
      s.urng[c * RS + 0] = u0;
      s.crng[c * RS + 0] = cum_b[c];
      if (has_ps && T > 0) s.prng[c * RS + 0] = ps_b[c] * kLog2e;
      if (store && j == 0) p.val[((size_t)b * (T + 1)) * C + c] = 0.0f;
      if (len == 0) p.fin[(size_t)b * C + c] = 0.0f;
    }
    if (tid == 0) {
      if (store && j == 0) p.lvl[(size_t)b * (T + 1)] = 0.0;
      if (len == 0) p.fin_lvl[b] = 0.0;
    }
    for (int k = tid; k <= Kmax; k += NT) s.dlt[k] = 0.0f;
  } else {
    // positions t_start - i, i in [0, Kmax)
    for (int idx = tid; idx < Kmax * C; idx += NT) {
      const int i = idx / C, cc = idx % C;
      const int pos = t_start - i;
      const int slot = pos % RS;
      s.urng[cc * RS + slot] = (mode == 1) ? 0.0f : init_st[(size_t)i * C + cc];
      s.crng[cc * RS + slot] = cum_b[(size_t)pos * C + cc];
      if (has_ps) s.prng[cc * RS + slot] = ps_b[(size_t)pos * C + cc] * kLog2e;
    }
    for (int i = tid; i < Kmax; i += NT) s.lring[(t_start - i) % RS] = (mode == 1) ? 0.0 : init_lv[i];
    const double l0 = (mode == 1) ? 0.0 : init_lv[0];
    for (int k = tid; k <= Kmax; k += NT)
      s.dlt[k] = (k <= 1 || mode == 1) ? 0.0f : (float)(init_lv[k - 1] - l0);
  }
  double lvl_prev = (mode == 2) ? init_lv[0] : 0.0;
  float cur_cum = (t_start + 1 <= T) ? cum_b[(size_t)(t_start + 1) * C + c] : 0.0f;
  float cur_pe = (has_pe && t_start < T) ? pe_b[(size_t)t_start * C + c] * kLog2e : 0.0f;
  __syncthreads();

  const int rec_spec = (mode == 1) ? t_lo : -1;
  for (int t = t_start + 1; t <= t_hi; ++t) {
    // prefetch next-step operands
    const float nxt_cum = (t + 1 <= T) ? cum_b[(size_t)(t + 1) * C + c] : 0.0f;
    const float nxt_pe = (has_pe && t < T) ? pe_b[(size_t)t * C + c] * kLog2e : 0.0f;
    const float cur_ps = (has_ps && t < T) ? ps_b[(size_t)t * C + c] * kLog2e : 0.0f;
    const int kcap = (mode == 0) ? min(Kmax, t) : Kmax;
    const int base = t % RS;
    const float* ur = s.urng + c * RS;
    const float* cr = s.crng + c * RS;
    const float* pr = s.prng + c * RS;
    const float* dr = s.dbt + c * (Kmax + 1);

    // ---- pull over durations ----
    Acc<LOGSR> acc;
    for (int k0 = 1 + lj; k0 <= kcap; k0 += 8 * J) {
      float xs[8];
      int n = 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + u * J;
        if (k <= kcap) {
          const int slot = wrap_slot(base - k, RS);
          float rest = dr[k] + s.dlt[k] + ur[slot];
          if (has_ps) rest += pr[slot];
          xs[u] = fmaf(cur_cum - cr[slot], kLog2e, rest);
          n = u + 1;
        }
      }
      acc.template add<8>(xs, n);
    }
    float a2 = acc.template reduce<J>();
    if (has_pe) a2 += cur_pe;

    // ---- normaliser: max over labels ----
    float wm = a2;
    for (int m = J; m < 64; m <<= 1) wm = fmax2(wm, __shfl_xor(wm, m, 64));
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
    // level differences for the next step: dlt[k] = lvl[t+1-k] - lvl[t]
    for (int k = tid + 1; k <= Kmax; k += NT)
      s.dlt[k] = (k == 1) ? 0.0f : (float)(s.lring[wrap_slot(base + 1 - k, RS)] - lvl_t);
    // ---- label mix: u[t,c] = (+)_{c'} alpha-hat[t,c'] + trans[c',c] ----
    const float u2 = label_mix<J, LOGSR>(s.row, s.trt, c, lj, C, mx);
    if (cval && lj == 0) {
      s.urng[c * RS + base] = u2;
      s.crng[c * RS + base] = cur_cum;
      if (has_ps) s.prng[c * RS + base] = cur_ps;
    }
    if (tid == 0) s.lring[base] = lvl_t;
    lvl_prev = lvl_t;
    cur_cum = nxt_cum;
    cur_pe = nxt_pe;
    __syncthreads();  // C
    // ---- boundary states for verification ----
    const bool rec_end = (t == t_hi) && (t_hi < len);
    if (t == rec_spec || rec_end) {
      float* st = (t == rec_spec ? p.st_spec : p.st_end) + (size_t)item * Kmax * C;
      double* lv = (t == rec_spec ? p.lv_spec : p.lv_end) + (size_t)item * Kmax;
      for (int idx = tid; idx < Kmax * C; idx += NT) {
        const int i = idx / C, cc = idx % C;
        st[idx] = s.urng[cc * RS + wrap_slot(base - i, RS)];
      }
      for (int i = tid; i < Kmax; i += NT) lv[i] = s.lring[wrap_slot(base - i, RS)];
    }
  }
}

// ============================================================================
// backward chunk (beta)
// mode 0: exact from position len; mode 1: speculative from t_hi + W;
// mode 2: exact from the state at t_hi given in (init_st, init_lv).
// Owned positions: [t_lo, t_hi) plus len for the last chunk.
// ============================================================================
template <int J, bool LOGSR, bool GR>
__device__ void backward_chunk(const ScanParams& p, char* smem_base, int b, int j, int mode,
                               const float* init_st, const double* init_lv) {
  const int C = p.C, Kmax = p.Kmax, RS = p.RS, T = p.T;
  const int len = seq_len(p, b);
  const int t_lo = j * p.Lc;
  const int jl = bwd_last_chunk(p, len);
  const int t_hi = (j == jl) ? len : (j + 1) * p.Lc;
  const int item = b * p.P + j;
  const bool has_ps = p.ps != nullptr, has_pe = p.pe != nullptr;
  Smem s = carve_scan_smem(smem_base, p, item, has_pe, GR);
  const int tid = threadIdx.x, NT = blockDim.x;
  const int c_raw = tid / J, lj = tid % J;
  const bool cval = c_raw < C;
  const int c = cval ? c_raw : C - 1;
  const int nw = (NT + 63) >> 6, wid = tid >> 6;
  const float* cum_b = p.cum + (size_t)b * (T + 1) * C;
  const float* ps_b = has_ps ? p.ps + (size_t)b * T * C : nullptr;
  const float* pe_b = has_pe ? p.pe + (size_t)b * T * C : nullptr;
  const bool store = p.val != nullptr;

  load_constants(p, s, false);
  const int t_start = mode == 0 ? len : (mode == 1 ? t_hi + p.W : t_hi);
  if (mode == 0) {
    if (cval && lj == 0) {
      s.urng[c * RS + len % RS] = 0.0f;
      s.crng[c * RS + len % RS] = cum_b[(size_t)len * C + c];
      if (store) p.val[((size_t)b * (T + 1) + len) * C + c] = 0.0f;
    }
    if (tid == 0) {
      s.lring[len % RS] = 0.0;
      if (store) p.lvl[(size_t)b * (T + 1) + len] = 0.0;
    }
    for (int k = tid; k <= Kmax; k += NT) s.dlt[k] = 0.0f;
  } else {
    for (int idx = tid; idx < Kmax * C; idx += NT) {
      const int i = idx / C, cc = idx % C;
      const int pos = t_start + i;
      const int slot = pos % RS;
      s.urng[cc * RS + slot] = (mode == 1) ? 0.0f : init_st[(size_t)i * C + cc];
      s.crng[cc * RS + slot] = cum_b[(size_t)pos * C + cc];
    }
    for (int i = tid; i < Kmax; i += NT) s.lring[(t_start + i) % RS] = (mode == 1) ? 0.0 : init_lv[i];
    const double l0 = (mode == 1) ? 0.0 : init_lv[0];
    // dlt[k] = lvl[t_start - 1 + k] - lvl[t_start]
    for (int k = tid; k <= Kmax; k += NT)
      s.dlt[k] = (k <= 1 || mode == 1) ? 0.0f : (float)(init_lv[k - 1] - l0);
  }
  // proj_end ring holds positions [t, t+Kmax-1] during step t (segment ends t+k-1)
  if (has_pe) {
    for (int idx = tid; idx < Kmax * C; idx += NT) {
      const int i = idx / C, cc = idx % C;
      const int pos = t_start - 1 + i;
      if (pos >= 0 && pos < T && pos < len) s.prng[cc * RS + pos % RS] = pe_b[(size_t)pos * C + cc] * kLog2e;
    }
  }
  double lvl_next = (mode == 2) ? init_lv[0] : 0.0;
  float cur_cum = (t_start >= 1) ? cum_b[(size_t)(t_start - 1) * C + c] : 0.0f;
  __syncthreads();

  const int rec_spec = (mode == 1) ? t_hi : -1;
  const int rec_end = (j >= 1) ? t_lo : -1;
  for (int t = t_start - 1; t >= t_lo; --t) {
    const float nxt_cum = (t >= 1) ? cum_b[(size_t)(t - 1) * C + c] : 0.0f;
    const float nxt_pe = (has_pe && t >= 1) ? pe_b[(size_t)(t - 1) * C + c] * kLog2e : 0.0f;
    const float cur_ps = has_ps ? ps_b[(size_t)t * C + c] * kLog2e : 0.0f;
    const int kcap = (mode == 0) ? min(Kmax, len - t) : Kmax;
    const int base = t % RS;
    const float* ur = s.urng + c * RS;
    const float* cr = s.crng + c * RS;
    const float* pr = s.prng + c * RS;
    const float* dr = s.dbt + c * (Kmax + 1);

    // ---- pull: w[t,c] = (+)_k seg(t,k,c) + beta[t+k,c] ----
    Acc<LOGSR> acc;
    for (int k0 = 1 + lj; k0 <= kcap; k0 += 8 * J) {
      float xs[8];
      int n = 0;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int k = k0 + u * J;
        if (k <= kcap) {
          int slot = base + k;
          if (slot >= RS) slot -= RS;
          float rest = dr[k] + s.dlt[k] + ur[slot];
          if (has_pe) {
            const int ps_slot = slot == 0 ? RS - 1 : slot - 1;
            rest += pr[ps_slot];
          }
          xs[u] = fmaf(cr[slot] - cur_cum, kLog2e, rest);
          n = u + 1;
        }
      }
      acc.template add<8>(xs, n);
    }
    float w2 = acc.template reduce<J>();
    if (has_ps) w2 += cur_ps;

    float wm = w2;
    for (int m = J; m < 64; m <<= 1) wm = fmax2(wm, __shfl_xor(wm, m, 64));
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
      s.urng[c * RS + base] = b2;
      s.crng[c * RS + base] = cur_cum;
      if (has_pe && t >= 1) s.prng[c * RS + wrap_slot(base - 1, RS)] = nxt_pe;
    }
    if (tid == 0) {
      if (store && owned) p.lvl[(size_t)b * (T + 1) + t] = lvl_t;
      s.lring[base] = lvl_t;
    }
    // dlt for step t-1: lvl[t-1+k] - lvl[t]
    for (int k = tid + 1; k <= Kmax; k += NT) {
      int slot = base - 1 + k;
      if (slot >= RS) slot -= RS;
      s.dlt[k] = (k == 1) ? 0.0f : (float)(s.lring[slot] - lvl_t);
    }
    lvl_next = lvl_t;
    cur_cum = nxt_cum;
    __syncthreads();  // C
    if (t == rec_spec || t == rec_end) {
      float* st = (t == rec_spec ? p.st_spec : p.st_end) + (size_t)item * Kmax * C;
      double* lv = (t == rec_spec ? p.lv_spec : p.lv_end) + (size_t)item * Kmax;
      for (int idx = tid; idx < Kmax * C; idx += NT) {
        const int i = idx / C, cc = idx % C;
        int slot = base + i;
        if (slot >= RS) slot -= RS;
        st[idx] = s.urng[cc * RS + slot];
      }
      for (int i = tid; i < Kmax; i += NT) {
        int slot = base + i;
        if (slot >= RS) slot -= RS;
        lv[i] = s.lring[slot];
      }
    }
  }
}

__device__ inline bool fwd_spec(const ScanParams& p, int j) { return j >= 1 && j * p.Lc - p.W >= p.Kmax - 1; }
__device__ inline bool bwd_spec(const ScanParams& p, int j, int len) {
  const int jl = bwd_last_chunk(p, len);
  return j < jl && (j + 1) * p.Lc + p.W + p.Kmax - 1 <= len;
}

template <int J, bool LOGSR, bool GR>
__global__ void __launch_bounds__(512) scan_fwd_kernel(ScanParams p) {
  extern __shared__ __align__(16) char smem[];
  const int b = blockIdx.x / p.P, j = blockIdx.x % p.P;
  const int len = seq_len(p, b);
  const int item = b * p.P + j;
  if (j > 0 && j * p.Lc >= len) {
    if (threadIdx.x == 0) p.status[item] = -1;  // empty chunk
    return;
  }
  const int mode = fwd_spec(p, j) ? 1 : 0;
  if (threadIdx.x == 0) p.status[item] = mode;
  forward_chunk<J, LOGSR, GR>(p, smem, b, j, mode, nullptr, nullptr);
}

template <int J, bool LOGSR, bool GR>
__global__ void __launch_bounds__(512) scan_bwd_kernel(ScanParams p) {
  extern __shared__ __align__(16) char smem[];
  const int b = blockIdx.x / p.P, j = blockIdx.x % p.P;
  const int len = seq_len(p, b);
  const int item = b * p.P + j;
  if (j > bwd_last_chunk(p, len)) {
    if (threadIdx.x == 0) p.status[item] = -1;
    return;
  }
  const int mode = bwd_spec(p, j, len) ? 1 : 0;
  if (threadIdx.x == 0) p.status[item] = mode;
  backward_chunk<J, LOGSR, GR>(p, smem, b, j, mode, nullptr, nullptr);
}

// Sequential verification / repair of a sequence's chunks (one block per sequence).
template <int J, bool LOGSR, bool GR>
__global__ void __launch_bounds__(512) fwd_fixup_kernel(ScanParams p) {
  extern __shared__ __align__(16) char smem[];
  const int b = blockIdx.x;
  const int len = seq_len(p, b);
  const ScanLds L = scan_lds_layout(p.C, p.Kmax, p.RS, p.ps != nullptr, GR);
  double* red = reinterpret_cast<double*>(smem + L.red);
  const int Kmax = p.Kmax, C = p.C;
  const int nch = len == 0 ? 1 : (len + p.Lc - 1) / p.Lc;
  double F = 0.0;
  int n_re = 0;
  if (threadIdx.x == 0) p.offs[(size_t)b * p.P] = 0.0;
  for (int j = 1; j < nch; ++j) {
    const int item = b * p.P + j;
    if (!fwd_spec(p, j)) {
      F = 0.0;  // chunk ran exactly from position 0
    } else {
      const size_t e = (size_t)(item - 1), sp = (size_t)item;
      double hi = -1e300, lo = 1e300;
      for (int idx = threadIdx.x; idx < Kmax * C; idx += blockDim.x) {
        const int i = idx / C;
        const float a = p.st_end[e * Kmax * C + idx], bb = p.st_spec[sp * Kmax * C + idx];
        if (a < -1e8f && bb < -1e8f) continue;
        const double d = (p.lv_end[e * Kmax + i] - p.lv_spec[sp * Kmax + i]) + ((double)a - (double)bb);
        hi = fmax(hi, d);
        lo = fmin(lo, d);
      }
      double dmax, dmin;
      block_minmax(hi, lo, red, dmax, dmin);
      if (dmax - dmin <= (double)p.tol) {
        F += 0.5 * (dmax + dmin);
      } else {
        forward_chunk<J, LOGSR, GR>(p, smem, b, j, 2, p.st_end + e * Kmax * C, p.lv_end + e * Kmax);
        __syncthreads();
        ++n_re;
        if (threadIdx.x == 0) p.status[item] = 2;
      }
    }
    if (threadIdx.x == 0) p.offs[(size_t)item] = F;
  }
  __syncthreads();
  // partition from the final row
  if (threadIdx.x < 64) {
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
}

template <int J, bool LOGSR, bool GR>
__global__ void __launch_bounds__(512) bwd_fixup_kernel(ScanParams p) {
  extern __shared__ __align__(16) char smem[];
  const int b = blockIdx.x;
  const int len = seq_len(p, b);
  const ScanLds L = scan_lds_layout(p.C, p.Kmax, p.RS, p.pe != nullptr, GR);
  double* red = reinterpret_cast<double*>(smem + L.red);
  const int Kmax = p.Kmax, C = p.C;
  const int jl = bwd_last_chunk(p, len);
  double F = 0.0;
  int n_re = 0;
  if (threadIdx.x == 0) p.offs[(size_t)b * p.P + jl] = 0.0;
  for (int j = jl - 1; j >= 0; --j) {
    const int item = b * p.P + j;
    if (!bwd_spec(p, j, len)) {
      F = 0.0;
    } else {
      const size_t e = (size_t)(item + 1), sp = (size_t)item;
      double hi = -1e300, lo = 1e300;
      for (int idx = threadIdx.x; idx < Kmax * C; idx += blockDim.x) {
        const int i = idx / C;
        const float a = p.st_end[e * Kmax * C + idx], bb = p.st_spec[sp * Kmax * C + idx];
        if (a < -1e8f && bb < -1e8f) continue;
        const double d = (p.lv_end[e * Kmax + i] - p.lv_spec[sp * Kmax + i]) + ((double)a - (double)bb);
        hi = fmax(hi, d);
        lo = fmin(lo, d);
      }
      double dmax, dmin;
      block_minmax(hi, lo, red, dmax, dmin);
      if (dmax - dmin <= (double)p.tol) {
        F += 0.5 * (dmax + dmin);
      } else {
        backward_chunk<J, LOGSR, GR>(p, smem, b, j, 2, p.st_end + e * Kmax * C, p.lv_end + e * Kmax);
        __syncthreads();
        ++n_re;
        if (threadIdx.x == 0) p.status[item] = 2;
      }
    }
    if (threadIdx.x == 0) p.offs[(size_t)item] = F;
  }
  if (threadIdx.x == 0 && p.recomputed != nullptr) p.recomputed[b] = n_re;
}

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

template <int J, bool LOGSR, bool GR>
int launch_dir(const Plan& pl, const ScanParams& p, bool forward, hipStream_t st) {
  const size_t lds = pl.scan_lds;
  if (forward) {
    auto k1 = scan_fwd_kernel<J, LOGSR, GR>;
    auto k2 = fwd_fixup_kernel<J, LOGSR, GR>;
    hipError_t e = hipFuncSetAttribute((const void*)k1, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute((const void*)k2, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k1, dim3(pl.B * pl.P), dim3(pl.NT), lds, st, p);
    hipLaunchKernelGGL(k2, dim3(pl.B), dim3(pl.NT), lds, st, p);
  } else {
    auto k1 = scan_bwd_kernel<J, LOGSR, GR>;
    auto k2 = bwd_fixup_kernel<J, LOGSR, GR>;
    hipError_t e = hipFuncSetAttribute((const void*)k1, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    e = hipFuncSetAttribute((const void*)k2, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(k1, dim3(pl.B * pl.P), dim3(pl.NT), lds, st, p);
    hipLaunchKernelGGL(k2, dim3(pl.B), dim3(pl.NT), lds, st, p);
  }
  if (p.lvl != nullptr) {
    const int per = 256;
    int gx = (pl.T + 1 + per - 1) / per;
    if (gx > 1024) gx = 1024;
    hipLaunchKernelGGL(apply_offsets_kernel, dim3(gx, pl.B), dim3(per), 0, st, p, forward ? 1 : 0);
  }
  return hipGetLastError();
}

template <bool LOGSR, bool GR>
int launch_j(const Plan& pl, const ScanParams& p, bool fwd, hipStream_t st) {
  switch (pl.J) {
    case 1: return launch_dir<1, LOGSR, GR>(pl, p, fwd, st);
    case 2: return launch_dir<2, LOGSR, GR>(pl, p, fwd, st);
    case 4: return launch_dir<4, LOGSR, GR>(pl, p, fwd, st);
    case 8: return launch_dir<8, LOGSR, GR>(pl, p, fwd, st);
    case 16: return launch_dir<16, LOGSR, GR>(pl, p, fwd, st);
    case 32: return launch_dir<32, LOGSR, GR>(pl, p, fwd, st);
    case 64: return launch_dir<64, LOGSR, GR>(pl, p, fwd, st);
    default: return (int)hipErrorInvalidValue;
  }
}

int launch_any(const Plan& pl, const ScanParams& p, int semiring, bool fwd, hipStream_t st) {
  if (semiring == kLog) {
    return pl.global_rings ? launch_j<true, true>(pl, p, fwd, st) : launch_j<true, false>(pl, p, fwd, st);
  }
  return pl.global_rings ? launch_j<false, true>(pl, p, fwd, st) : launch_j<false, false>(pl, p, fwd, st);
}

}  // namespace

int launch_scan_forward(const Plan& pl, const ScanParams& p, int semiring, hipStream_t s) {
  return launch_any(pl, p, semiring, true, s);
}
int launch_scan_backward(const Plan& pl, const ScanParams& p, int semiring, hipStream_t s) {
  return launch_any(pl, p, semiring, false, s);
}

}  // namespace tsm
