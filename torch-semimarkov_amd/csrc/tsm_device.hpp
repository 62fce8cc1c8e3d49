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

// Hardware base-2 exponential (v_exp_f32).  Measured on MI355X against fp64:
// mean relative error -3.4e-9, rms 2.6e-8 over [-20, 0].
__device__ __forceinline__ float exp2_hw(float x) { return __builtin_amdgcn_exp2f(x); }

// Base-2 logarithm.  v_log_f32 alone is biased, and more so for larger
// arguments (measured mean error against fp64: -8e-9 on [0.5, 1), -1.8e-7 on
// [4, 32), -3.4e-7 on [1, 512)).  The scans take two logarithms of sums of up
// to a few hundred terms per step, so that bias accumulated along the level
// chains (about -1e-7 log2 units per step).  Here x = m * 2^e is split exactly
// (v_frexp_mant / v_frexp_exp, m in [0.5, 1)) and only m goes through v_log_f32;
// e is added exactly, with the sum rounded to nearest.  x = 0 gives -inf (m = 0),
// x = +inf gives +inf, NaN stays NaN.
__device__ __forceinline__ float log2_hw(float x) {
  const float e = (float)__builtin_amdgcn_frexp_expf(x);
  return e + __builtin_amdgcn_logf(__builtin_amdgcn_frexp_mantf(x));
}

__device__ __forceinline__ float fmax2(float a, float b) { return __builtin_fmaxf(a, b); }

// ----------------------------------------------------------------------------
// Reductions inside a group of G consecutive lanes (G a power of two, G <= 64).
// Groups never straddle a wavefront because 64 % G == 0.  Every lane receives
// the group result.  Inside a 16-lane row the partner values come from DPP
// (quad_perm xor1 / xor2, row_half_mirror, row_mirror: after the quad steps all
// lanes of a quad agree, so mirroring pairs whole quads / half rows); across
// rows v_permlane16_swap / v_permlane32_swap exchange rows, and for a
// symmetric op, op(pair.first, pair.second) equals op(x[lane], x[lane^16]) (or
// ^32) on every lane.  No LDS traffic and no waits on the LDS pipeline.
// ----------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}

constexpr int kDppXor1 = 0xB1;         // quad_perm(1,0,3,2)
constexpr int kDppXor2 = 0x4E;         // quad_perm(2,3,0,1)
constexpr int kDppHalfMirror = 0x141;  // row_half_mirror
constexpr int kDppMirror = 0x140;      // row_mirror

struct OpMax {
  __device__ __forceinline__ float operator()(float a, float b) const { return fmax2(a, b); }
};
struct OpSum {
  __device__ __forceinline__ float operator()(float a, float b) const { return a + b; }
};

template <int G, typename Op>
__device__ __forceinline__ float group_reduce(float v, Op op) {
  if constexpr (G >= 2) v = op(v, dpp_f<kDppXor1>(v));
  if constexpr (G >= 4) v = op(v, dpp_f<kDppXor2>(v));
  if constexpr (G >= 8) v = op(v, dpp_f<kDppHalfMirror>(v));
  if constexpr (G >= 16) v = op(v, dpp_f<kDppMirror>(v));
  if constexpr (G >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
    v = op(__int_as_float(r[0]), __int_as_float(r[1]));
  }
  if constexpr (G >= 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    v = op(__int_as_float(r[0]), __int_as_float(r[1]));
  }
  return v;
}

// max(v, DPP-permuted v) as one v_max_f32 with a DPP source.  fmaxf of a DPP
// move costs four instructions (old-value fill, move, canonicalising max,
// max); v_max_f32 already returns the non-NaN operand, as fmaxf does.  The
// s_nop gives the two wait states a DPP read needs after a VALU write, which
// the compiler does not track across inline asm.  All lanes must be active
// (as for every group reduction here).
template <int CTRL>
__device__ __forceinline__ float dpp_max(float v) {
  float r;
  if constexpr (CTRL == 0xB1) {
    asm("s_nop 1\n\tv_max_f32_dpp %0, %1, %1 quad_perm:[1,0,3,2] row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(r) : "v"(v));
  } else if constexpr (CTRL == 0x4E) {
    asm("s_nop 1\n\tv_max_f32_dpp %0, %1, %1 quad_perm:[2,3,0,1] row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(r) : "v"(v));
  } else if constexpr (CTRL == 0x141) {
    asm("s_nop 1\n\tv_max_f32_dpp %0, %1, %1 row_half_mirror row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(r) : "v"(v));
  } else {
    static_assert(CTRL == 0x140, "dpp_max: unsupported DPP pattern");
    asm("s_nop 1\n\tv_max_f32_dpp %0, %1, %1 row_mirror row_mask:0xf bank_mask:0xf bound_ctrl:1"
        : "=v"(r) : "v"(v));
  }
  return r;
}

template <int G>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (G >= 2) v = dpp_max<kDppXor1>(v);
  if constexpr (G >= 4) v = dpp_max<kDppXor2>(v);
  if constexpr (G >= 8) v = dpp_max<kDppHalfMirror>(v);
  if constexpr (G >= 16) v = dpp_max<kDppMirror>(v);
  if constexpr (G >= 32) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_int(v), __float_as_int(v), false, false);
    v = fmax2(__int_as_float(r[0]), __int_as_float(r[1]));
  }
  if constexpr (G >= 64) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_int(v), __float_as_int(v), false, false);
    v = fmax2(__int_as_float(r[0]), __int_as_float(r[1]));
  }
  return v;
}

template <int G>
__device__ __forceinline__ float group_sum(float v) {
  return group_reduce<G>(v, OpSum{});
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

// a + (lane (i-1) mod 16 of the row of `rot`): the end-sum slide of the fused
// marginals.  A DPP move (row_ror:1) left to the compiler, so it schedules the
// wait states a DPP read needs after a VALU write (only where the schedule
// needs them) and fuses a product added here into an FMA after the move.  All
// lanes are active.
__device__ __forceinline__ float add_row_ror1(float rot, float a) {
  return a + __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(rot), 0x121, 0xf, 0xf, true));
}

// CJ source labels per lane in the label mix (C <= CJ * J; the launchers pick 2
// when C <= 2J, else 4).
// Max with the index of the first maximum: ties go to the smaller index.
struct ValIdx {
  float v;
  int i;
};

__device__ __forceinline__ ValIdx better_first(ValIdx a, float ov, int oi) {
  if (ov > a.v || (ov == a.v && oi < a.i)) return ValIdx{ov, oi};
  return a;
}

template <int G>
__device__ __forceinline__ ValIdx group_argmax_first(ValIdx a) {
  if constexpr (G >= 2) a = better_first(a, dpp_f<kDppXor1>(a.v), dpp_i<kDppXor1>(a.i));
  if constexpr (G >= 4) a = better_first(a, dpp_f<kDppXor2>(a.v), dpp_i<kDppXor2>(a.i));
  if constexpr (G >= 8) a = better_first(a, dpp_f<kDppHalfMirror>(a.v), dpp_i<kDppHalfMirror>(a.i));
  if constexpr (G >= 16) a = better_first(a, dpp_f<kDppMirror>(a.v), dpp_i<kDppMirror>(a.i));
  if constexpr (G >= 32) {
    const auto rv = __builtin_amdgcn_permlane16_swap(__float_as_int(a.v), __float_as_int(a.v), false, false);
    const auto ri = __builtin_amdgcn_permlane16_swap(a.i, a.i, false, false);
    a = better_first(ValIdx{__int_as_float(rv[0]), (int)ri[0]}, __int_as_float(rv[1]), (int)ri[1]);
  }
  if constexpr (G >= 64) {
    const auto rv = __builtin_amdgcn_permlane32_swap(__float_as_int(a.v), __float_as_int(a.v), false, false);
    const auto ri = __builtin_amdgcn_permlane32_swap(a.i, a.i, false, false);
    a = better_first(ValIdx{__int_as_float(rv[0]), (int)ri[0]}, __int_as_float(rv[1]), (int)ri[1]);
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
