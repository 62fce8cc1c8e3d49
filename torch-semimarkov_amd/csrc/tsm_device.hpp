// Device-side helpers shared by the semi-Markov scan kernels (gfx950 / CDNA4).
//
// Numerics used by the log-semiring kernels:
//   * everything is carried in base-2 log units ("log2 domain"): an input score
//     x (natural log units) becomes x * log2(e) once, so every exponential is
//     a single hardware v_exp_f32 and every logarithm a single v_log_f32;
//   * per-position state is stored normalised (max over labels = 0) in fp32,
//     with the per-position normaliser ("level") accumulated in fp64, so the
//     fp32 payload stays O(10) however long the sequence is.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace tsm {

constexpr float kNegInf = -1e9f;                      // reference sentinel (constants.py:10)
constexpr float kLog2e = 1.4426950408889634f;         // log2(e)
constexpr double kLn2 = 0.6931471805599453;           // ln(2)
constexpr float kMinusInf = -__builtin_inff();

// Hardware base-2 exponential / logarithm (v_exp_f32 / v_log_f32, ~1 ulp).
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float log2_hw(float x) { return __builtin_amdgcn_logf(x); }

__device__ __forceinline__ float fmax2(float a, float b) { return __builtin_fmaxf(a, b); }

// ----------------------------------------------------------------------------
// Reductions inside a group of G consecutive lanes (G a power of two, G <= 64).
// Groups never straddle a wavefront because 64 % G == 0.
// ----------------------------------------------------------------------------
template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int m = 1; m < G; m <<= 1) v = fmax2(v, __shfl_xor(v, m, 64));
  return v;
}

template <int G>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int m = 1; m < G; m <<= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Log-sum-exp (base 2) of per-lane partials (m, s), where each lane holds
// sum_i 2^(x_i - m) = s.  Returns log2(sum over the group of 2^x_i).
template <int G>
__device__ __forceinline__ float group_lse2(float m, float s) {
  const float M = group_max<G>(m);
  float t = (m == kMinusInf) ? 0.0f : s * exp2_hw(m - M);
  t = group_sum<G>(t);
  return M + log2_hw(t);
}

// Max with the index of the first maximum: ties go to the smaller index.
struct ValIdx {
  float v;
  int i;
};

template <int G>
__device__ __forceinline__ ValIdx group_argmax_first(ValIdx a) {
#pragma unroll
  for (int m = 1; m < G; m <<= 1) {
    float ov = __shfl_xor(a.v, m, 64);
    int oi = __shfl_xor(a.i, m, 64);
    if (ov > a.v || (ov == a.v && oi < a.i)) {
      a.v = ov;
      a.i = oi;
    }
  }
  return a;
}

// Online log-sum-exp accumulator in base 2 over a lane's terms, processed in
// register batches so the running maximum is rescaled once per batch.
struct Lse2Acc {
  float m = kMinusInf;
  float s = 0.0f;
  template <int N>
  __device__ __forceinline__ void add_batch(const float (&x)[N], int n) {
    if (n <= 0) return;
    float bm = x[0];
#pragma unroll
    for (int i = 1; i < N; ++i)
      if (i < n) bm = fmax2(bm, x[i]);
    const float nm = fmax2(m, bm);
    float acc = (m == kMinusInf) ? 0.0f : s * exp2_hw(m - nm);
#pragma unroll
    for (int i = 0; i < N; ++i)
      if (i < n) acc += exp2_hw(x[i] - nm);
    m = nm;
    s = acc;
  }
};

__device__ __forceinline__ int wrap_slot(int slot, int RS) { return slot < 0 ? slot + RS : slot; }

}  // namespace tsm
