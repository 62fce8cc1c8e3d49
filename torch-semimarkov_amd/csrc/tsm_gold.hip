// Gold-path score: the score of the segmentation implied by per-position
// labels, and its gradients, for gfx950.
//
// Semantics (reference helpers.py:365-544, score_gold_vectorized): segments are
// the maximal runs of equal labels inside [0, len); a segment [s, e] with
// label c contributes
//   cum[e+1, c] - cum[s, c] + duration_bias[clamp(e-s+1, 1, K-1), c] + transition[c_prev, c]
// with no transition for the first segment (torch.clamp with min > max gives
// max, so K = 1 uses row 0); for T == 1 the duration row is 1 (:410-419),
// clamped here to the table.
//
// No segment list is built.  Every position p decides locally whether it
// starts a segment (p == 0 or label[p-1] != label[p]) and whether it ends one
// (p == len-1 or label[p+1] != label[p]); a start adds -cum[p, c] and the
// transition from label[p-1], an end adds cum[p+1, c] and the duration bias,
// whose row needs the run length only up to K-1: an end looks back at most
// K-2 labels.  The total work is O(T) per sequence, with no scan and no host
// synchronisation (the reference walks the batch in Python with .item()).
//
// Forward: one block per (sequence, TB positions); labels staged in LDS as
// int32 with the K-2 lookback; per-position terms summed in fp64 and reduced
// per block, then per sequence in a fixed order (deterministic).  A label
// outside [0, C) inside a sequence makes that sequence's score NaN (it is
// never used as an index).
// Backward: grad_cum is written densely, one writer per element (+g at e+1
// of an end, -g at a start); segment and transition counts go to per-sequence
// integer histograms by global atomics (order-independent, so deterministic)
// and are weighted by grad_output in fp64 by a final reduction.

#include "tsm_device.hpp"
#include "tsm_internal.hpp"

namespace tsm {
namespace {

constexpr int kGoldNT = 256;
constexpr int kGoldTB = 2048;  // positions per block

__device__ inline int glen(const int64_t* lengths, int b, int T) {
  int64_t L = lengths[b];
  if (L < 0) L = 0;
  if (L > T) L = T;
  return (int)L;
}

// Duration-bias row of a segment of duration dur (>= 1).
__device__ inline int gold_row(int dur, const GoldParams& g) {
  if (g.T == 1) return g.Kdb > 1 ? 1 : 0;
  if (g.K <= 1) return 0;
  return dur < g.K - 1 ? dur : g.K - 1;
}

// Stages labels of positions [p0 - H, p0 + TB] (H = lookback) as int32; -1 for
// positions outside [0, len).  Returns the pointer to position p0.
__device__ inline const int* stage_labels(const GoldParams& g, int b, int p0, int len, int H, int* lab) {
  const int64_t* lb = g.labels + (size_t)b * g.T;
  for (int i = threadIdx.x; i < H + kGoldTB + 1; i += blockDim.x) {
    const int p = p0 - H + i;
    lab[i] = (p >= 0 && p < len) ? (int)lb[p] : -1;
  }
  __syncthreads();
  return lab + H;
}

// Run length (capped at K-1) of the run of label c ending at position p.
__device__ inline int run_length(const int* lp, int p, int c, int cap) {
  int d = 1;
  while (d < cap && p - d >= 0 && lp[-d] == c) ++d;
  return d;
}

__global__ void __launch_bounds__(kGoldNT) gold_partial_kernel(GoldParams g) {
  extern __shared__ __align__(16) char smem[];
  int* lab = reinterpret_cast<int*>(smem);
  __shared__ double red[kGoldNT / 64];
  __shared__ int bad_w[kGoldNT / 64];
  const int chunk = blockIdx.x % g.NCH, b = blockIdx.x / g.NCH;
  const int C = g.C, T = g.T;
  const int len = glen(g.lengths, b, T);
  const int p0 = chunk * kGoldTB;
  const int H = g.H;
  const int* lp = stage_labels(g, b, p0, len, H, lab);
  const float* em_b = g.emit != nullptr ? g.emit + (size_t)b * T * C : nullptr;
  const float* cum_b = em_b != nullptr ? nullptr : g.cum + (size_t)b * (T + 1) * C;
  const int cap = g.K - 1;
  double acc = 0.0;
  int bad = 0;
  const int p_end = min(p0 + kGoldTB, len);
  for (int p = p0 + threadIdx.x; p < p_end; p += blockDim.x) {
    const int i = p - p0;
    const int c = lp[i];
    if (c < 0 || c >= C) {
      bad = 1;
      continue;
    }
    const int cprev = (p > 0) ? lp[i - 1] : -1;
    const int cnext = (p + 1 < len) ? lp[i + 1] : -1;
    // emission input: a segment's content is the sum of its positions' scores
    if (em_b != nullptr) acc += (double)em_b[(size_t)p * C + c];
    if (p == 0 || cprev != c) {
      if (em_b == nullptr) acc -= (double)cum_b[(size_t)p * C + c];
      if (p > 0) {
        if (cprev < 0 || cprev >= C) bad = 1;
        else acc += (double)g.tr[(size_t)cprev * C + c];
      }
    }
    if (p == len - 1 || cnext != c) {
      const int dur = (g.T > 1 && cap > 1) ? run_length(lp + i, p, c, cap) : 1;
      if (em_b == nullptr) acc += (double)cum_b[(size_t)(p + 1) * C + c];
      acc += (double)g.db[(size_t)gold_row(dur, g) * C + c];
    }
  }
  // block reduction (fp64 sum, flag or)
  for (int m = 32; m >= 1; m >>= 1) {
    acc += __shfl_xor(acc, m, 64);
    bad |= __shfl_xor(bad, m, 64);
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    red[w] = acc;
    bad_w[w] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    double s = 0.0;
    int f = 0;
    for (int i = 0; i < kGoldNT / 64; ++i) {
      s += red[i];
      f |= bad_w[i];
    }
    g.part[(size_t)b * g.NCH + chunk] = s;
    g.bad[(size_t)b * g.NCH + chunk] = f;
  }
}

// score[b] = sum of the block partials in chunk order (NaN after a bad label).
__global__ void gold_finish_kernel(GoldParams g) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= g.B) return;
  double s = 0.0;
  int f = 0;
  for (int i = 0; i < g.NCH; ++i) {
    s += g.part[(size_t)b * g.NCH + i];
    f |= g.bad[(size_t)b * g.NCH + i];
  }
  g.score[b] = f ? __builtin_nanf("") : (float)s;
}

// grad_cum[b, p, c] = g_b * ([p-1 ends a segment of label c] - [p starts a segment of label c]).
__global__ void gold_grad_cum_kernel(GoldParams g) {
  const int C = g.C, T = g.T;
  const size_t n = (size_t)g.B * (T + 1) * C;
  if (g.emit_grad) {
    // emission input: d gold / d scores[b, p, c] = [p < len and labels[b, p] == c]
    const size_t m = (size_t)g.B * T * C;
    for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < m; idx += (size_t)gridDim.x * blockDim.x) {
      const int c = (int)(idx % C);
      const int p = (int)((idx / C) % T);
      const int b = (int)(idx / ((size_t)C * T));
      const bool on = p < glen(g.lengths, b, T) && g.labels[(size_t)b * T + p] == c;
      g.gcum[idx] = on ? g.gout[b] : 0.0f;
    }
    return;
  }
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (size_t)gridDim.x * blockDim.x) {
    const int c = (int)(idx % C);
    const int p = (int)((idx / C) % (T + 1));
    const int b = (int)(idx / ((size_t)C * (T + 1)));
    const int len = glen(g.lengths, b, T);
    const int64_t* lb = g.labels + (size_t)b * T;
    float v = 0.0f;
    if (p >= 1 && p <= len) {
      // position p-1 ends a segment of label c
      const int64_t l = lb[p - 1];
      if (l == c && (p == len || lb[p] != l)) v += 1.0f;
    }
    if (p < len) {
      const int64_t l = lb[p];
      if (l == c && (p == 0 || lb[p - 1] != l)) v -= 1.0f;
    }
    g.gcum[idx] = v * g.gout[b];
  }
}

// Per-sequence histograms: cnt[b][row*C + c] segments with duration row / label c,
// cnt[b][Kdb*C + c'*C + c] transitions c' -> c.
__global__ void __launch_bounds__(kGoldNT) gold_count_kernel(GoldParams g) {
  extern __shared__ __align__(16) char smem[];
  int* lab = reinterpret_cast<int*>(smem);
  const int chunk = blockIdx.x % g.NCH, b = blockIdx.x / g.NCH;
  const int C = g.C, T = g.T;
  const int len = glen(g.lengths, b, T);
  const int p0 = chunk * kGoldTB;
  const int* lp = stage_labels(g, b, p0, len, g.H, lab);
  int* cnt = g.cnt + (size_t)b * g.NHIST;
  const int cap = g.K - 1;
  const int p_end = min(p0 + kGoldTB, len);
  for (int p = p0 + threadIdx.x; p < p_end; p += blockDim.x) {
    const int i = p - p0;
    const int c = lp[i];
    if (c < 0 || c >= C) continue;
    const int cprev = (p > 0) ? lp[i - 1] : -1;
    const int cnext = (p + 1 < len) ? lp[i + 1] : -1;
    if (p > 0 && cprev != c && cprev >= 0 && cprev < C) atomicAdd(&cnt[g.Kdb * C + cprev * C + c], 1);
    if (p == len - 1 || cnext != c) {
      const int dur = (g.T > 1 && cap > 1) ? run_length(lp + i, p, c, cap) : 1;
      atomicAdd(&cnt[gold_row(dur, g) * C + c], 1);
    }
  }
}

__global__ void gold_zero_kernel(int* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

// grad_duration_bias / grad_transition = sum_b g_b * counts (fp64).
__global__ void gold_shared_kernel(GoldParams g) {
  const int idx = blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= g.NHIST) return;
  double s = 0.0;
  for (int b = 0; b < g.B; ++b) s += (double)g.gout[b] * (double)g.cnt[(size_t)b * g.NHIST + idx];
  const int ndb = g.Kdb * g.C;
  if (idx < ndb) g.gdb[idx] = (float)s;
  else g.gtr[idx - ndb] = (float)s;
}

inline size_t gold_lds(int H) { return sizeof(int) * (size_t)(H + kGoldTB + 1); }

}  // namespace

int gold_chunks(int T) { return (T + kGoldTB - 1) / kGoldTB; }

size_t gold_lds_bytes(int K) { return gold_lds(K > 3 ? K - 2 : 1); }

int launch_gold_score(const GoldParams& g0, hipStream_t s) {
  GoldParams g = g0;
  g.H = g.K > 3 ? g.K - 2 : 1;
  const size_t lds = gold_lds(g.H);
  hipError_t e = hipFuncSetAttribute((const void*)gold_partial_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)lds);
  if (e != hipSuccess) return e;
  {
    TimedLaunch tl(kKGold, s);
    hipLaunchKernelGGL(gold_partial_kernel, dim3(g.NCH * g.B), dim3(kGoldNT), lds, s, g);
    hipLaunchKernelGGL(gold_finish_kernel, dim3((g.B + 63) / 64), dim3(64), 0, s, g);
  }
  return hipGetLastError();
}

int launch_gold_backward(const GoldParams& g0, hipStream_t s) {
  GoldParams g = g0;
  g.H = g.K > 3 ? g.K - 2 : 1;
  const size_t lds = gold_lds(g.H);
  hipError_t e = hipFuncSetAttribute((const void*)gold_count_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                     (int)lds);
  if (e != hipSuccess) return e;
  TimedLaunch tl(kKGold, s);
  const size_t n = (size_t)g.B * (g.T + 1) * g.C;
  int gx = (int)((n + 255) / 256);
  if (gx > 8192) gx = 8192;
  hipLaunchKernelGGL(gold_grad_cum_kernel, dim3(gx), dim3(256), 0, s, g);
  const size_t nh = (size_t)g.B * g.NHIST;
  int gz = (int)((nh + 255) / 256);
  if (gz > 4096) gz = 4096;
  hipLaunchKernelGGL(gold_zero_kernel, dim3(gz), dim3(256), 0, s, g.cnt, nh);
  hipLaunchKernelGGL(gold_count_kernel, dim3(g.NCH * g.B), dim3(kGoldNT), lds, s, g);
  hipLaunchKernelGGL(gold_shared_kernel, dim3((g.NHIST + 255) / 256), dim3(256), 0, s, g);
  return hipGetLastError();
}

}  // namespace tsm
