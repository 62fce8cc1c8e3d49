// Exact Viterbi (max semiring) with backpointers (the backtrace is tsm_backtrace.hip).
//
// This kernel reproduces the reference's fp32 arithmetic operation for
// operation, so scores are bit-identical and segmentations match exactly:
//   edge  = (((cum[t,c]-cum[s,c]) + db[min(k,K-1),c]) (+ps[s,c]) (+pe[t-1,c])) + trans[c',c]
//   score = alpha[s,c'] + edge                       (streaming/pytorch_reference.py:86-111, 229)
//   alpha[t,c] = max_k max_c' score                  (:240-241)
// Ties follow nn.py:472-501: the smallest duration wins (strict '>' over k in
// ascending order), then the first source label (torch.max), and the
// backtrace starts from the first maximising final label (argmax).
// Raw (un-normalised) fp32 alpha values are kept, exactly as the reference.
//
// One workgroup per sequence; the K x C alpha ring lives in LDS.  Lanes of a
// label group split the durations; the transition row of the label sits in
// registers (CMAX >= C, a multiple of 8) when the group has at least 16 lanes.

#include "tsm_device.hpp"
#include "tsm_internal.hpp"

namespace tsm {
namespace {

struct VLds {
  size_t araw, crng, prng, dbn, trn, red, total;
};

// araw is position-major, [slot][c] with the odd row stride C|1: the source
// labels of one ring position are consecutive (immediate-offset loads) and the
// rows a label group reads at once fall on different banks.  crng / prng are
// label-major, [c][slot].
__host__ __device__ inline VLds vit_lds_layout(int C, int Kmax, int RS, int has_ps) {
  VLds L;
  size_t o = 0;
  const size_t ring = sizeof(float) * (size_t)C * RS;
  L.araw = o; o = align16(o + sizeof(float) * (size_t)(C | 1) * RS);
  L.crng = o; o = align16(o + ring);
  L.prng = o; o = align16(o + (has_ps ? ring : 0));
  L.dbn = o; o = align16(o + sizeof(float) * (size_t)C * (Kmax + 1));
  L.trn = o; o = align16(o + sizeof(float) * (size_t)C * C);
  L.red = o; o = align16(o + sizeof(float) * 64 + sizeof(int) * 64);
  L.total = o;
  return L;
}

template <int J, int CMAX>
__global__ void __launch_bounds__(1024) viterbi_kernel(ViterbiParams v) {
  extern __shared__ __align__(16) char smem[];
  const int b = blockIdx.x;
  const int C = v.C, K = v.K, Kmax = v.Kmax, RS = v.RS, T = v.T, CS = C | 1;
  int64_t L64 = v.lengths[b];
  const int len = (int)(L64 < 0 ? 0 : (L64 > T ? T : L64));
  const bool has_ps = v.ps != nullptr, has_pe = v.pe != nullptr;
  const VLds Ly = vit_lds_layout(C, Kmax, RS, has_ps);
  float* araw = reinterpret_cast<float*>(smem + Ly.araw);
  float* crng = reinterpret_cast<float*>(smem + Ly.crng);
  float* prng = reinterpret_cast<float*>(smem + Ly.prng);
  float* dbn = reinterpret_cast<float*>(smem + Ly.dbn);
  float* trn = reinterpret_cast<float*>(smem + Ly.trn);
  float* redv = reinterpret_cast<float*>(smem + Ly.red);
  int* redi = reinterpret_cast<int*>(smem + Ly.red + sizeof(float) * 64);

  const int tid = threadIdx.x, NT = blockDim.x;
  const int c_raw = tid / J, lj = tid % J;
  const bool cval = c_raw < C;
  const int c = cval ? c_raw : C - 1;
  const float* cum_b = v.cum + (size_t)b * (T + 1) * C;
  const float* ps_b = has_ps ? v.ps + (size_t)b * T * C : nullptr;
  const float* pe_b = has_pe ? v.pe + (size_t)b * T * C : nullptr;

  for (int idx = tid; idx < C * (Kmax + 1); idx += NT) {
    const int cc = idx / (Kmax + 1), k = idx % (Kmax + 1);
    const int di = k < K - 1 ? k : K - 1;
    dbn[idx] = v.db[(size_t)di * C + cc];
  }
  if (v.trows == 0) {
    for (int idx = tid; idx < C * C; idx += NT) {
      const int cd = idx / C, cs = idx % C;
      trn[idx] = v.trans[(size_t)cs * C + cd];  // [c_dst][c_src]
    }
  }
  for (int cc = tid; cc < C; cc += NT) {
    araw[cc] = 0.0f;  // alpha[0, :] = 0 (slot 0)
    crng[cc * RS] = cum_b[cc];
    if (has_ps && T > 0) prng[cc * RS] = ps_b[cc];
  }
  __syncthreads();
  float tr_reg[CMAX > 0 ? CMAX : 1];
  if constexpr (CMAX > 0) {
#pragma unroll
    for (int i = 0; i < CMAX; ++i) tr_reg[i] = trn[c * C + min(i, C - 1)];  // padding repeats the last label
  }
  const float* dr = dbn + c * (Kmax + 1);
  const float* cr = crng + c * RS;
  const float* pr = prng + c * RS;

  // this step's cumulative score and projections, loaded one step ahead
  float cum_n = len >= 1 ? cum_b[(size_t)C + c] : 0.0f;
  float pe_n = (has_pe && len >= 1) ? pe_b[c] : 0.0f;
  float ps_n = (has_ps && len >= 1 && T > 1) ? ps_b[(size_t)C + c] : 0.0f;
  for (int t = 1; t <= len; ++t) {
    const int kcap = (K == 1) ? 1 : min(K - 1, t);
    const int base = t % RS;
    const float cur_cum = cum_n;
    const float pe_t = pe_n;
    const float ps_t = ps_n;  // proj_start of position t (ring entry of position t)
    if (t < len) {
      cum_n = cum_b[(size_t)(t + 1) * C + c];
      if (has_pe) pe_n = pe_b[(size_t)t * C + c];
      if (has_ps && t + 1 < T) ps_n = ps_b[(size_t)(t + 1) * C + c];
    }
    float bv = kMinusInf;
    int bk = 0;
    for (int k = 1 + lj; k <= kcap; k += J) {
      const int slot = wrap_slot(base - k, RS);
      float e1 = (cur_cum - cr[slot]) + dr[k];
      if (has_ps) e1 = e1 + pr[slot];
      if (has_pe) e1 = e1 + pe_t;
      // max over source labels; the loads of a block are issued together (indices
      // past C repeat the last label's term, which leaves the max unchanged), and
      // four running maxima keep the max chain short (max is exact in any order)
      const float* arow = araw + (size_t)slot * CS;
      float m4[4] = {kMinusInf, kMinusInf, kMinusInf, kMinusInf};
      if (v.trows > 0) {
        // duration-dependent transitions: transition[k][c_src][c], from global memory
        const float* tk = v.trans + (size_t)k * C * C + c;
        for (int i0 = 0; i0 < C; i0 += 8) {
          float a[8], tt[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int i = min(i0 + u, C - 1);
            a[u] = arow[i];
            tt[u] = tk[(size_t)i * C];
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) m4[u & 3] = fmax2(m4[u & 3], a[u] + (e1 + tt[u]));
        }
      } else if constexpr (CMAX > 0) {
        float a[CMAX];
#pragma unroll
        for (int i = 0; i < CMAX; ++i) a[i] = arow[min(i, C - 1)];
#pragma unroll
        for (int i = 0; i < CMAX; ++i) m4[i & 3] = fmax2(m4[i & 3], a[i] + (e1 + tr_reg[i]));
      } else {
        const float* trow = trn + c * C;
        for (int i0 = 0; i0 < C; i0 += 8) {
          float a[8], tt[8];
#pragma unroll
          for (int u = 0; u < 8; ++u) {
            const int i = min(i0 + u, C - 1);
            a[u] = arow[i];
            tt[u] = trow[i];
          }
#pragma unroll
          for (int u = 0; u < 8; ++u) m4[u & 3] = fmax2(m4[u & 3], a[u] + (e1 + tt[u]));
        }
      }
      const float m = fmax2(fmax2(m4[0], m4[1]), fmax2(m4[2], m4[3]));
      if (m > bv) {
        bv = m;
        bk = k;
      }
    }
    ValIdx best = group_argmax_first<J>(ValIdx{bv, bk == 0 ? 0x7fffffff : bk});
    if (v.bp != nullptr) {
      // first source label attaining the max at the winning duration (a duration
      // in range even when no score was finite, e.g. NaN inputs: the index
      // addresses the transition table)
      const int ks = (best.i >= 1 && best.i <= kcap) ? best.i : 1;
      const int slot = wrap_slot(base - ks, RS);
      float e1 = (cur_cum - cr[slot]) + dr[ks];
      if (has_ps) e1 = e1 + pr[slot];
      if (has_pe) e1 = e1 + pe_t;
      float cv = kMinusInf;
      int ci = 0x7fffffff;
      const float* tk = v.trans + (size_t)ks * C * C + c;
      for (int i = lj; i < C; i += J) {
        const float x = araw[(size_t)slot * CS + i] + (e1 + (v.trows > 0 ? tk[(size_t)i * C] : trn[c * C + i]));
        if (x > cv) {
          cv = x;
          ci = i;
        }
      }
      const ValIdx cs = group_argmax_first<J>(ValIdx{cv, ci});
      if (cval && lj == 0) v.bp[((size_t)b * (T + 1) + t) * C + c] = (ks << 16) | cs.i;
    }
    // slot t % RS holds position t - RS, which step t never reads (RS >= Kmax+1),
    // so the ring can be updated without waiting for the other labels' reads.
    if (cval && lj == 0) {
      araw[(size_t)base * CS + c] = best.v;
      crng[c * RS + base] = cur_cum;
      if (has_ps && t < T) prng[c * RS + base] = ps_t;
    }
    __syncthreads();
  }
  // ---- score = max over labels of alpha[len]; first maximising label ----
  {
    const int slot = len % RS;
    float mv = kMinusInf;
    int mi = 0x7fffffff;
    for (int cc = tid; cc < C; cc += NT) {
      const float x = araw[(size_t)slot * CS + cc];
      if (x > mv || (x == mv && cc < mi)) {
        mv = x;
        mi = cc;
      }
    }
    ValIdx r = group_argmax_first<64>(ValIdx{mv, mi});
    if ((tid & 63) == 0) {
      redv[tid >> 6] = r.v;
      redi[tid >> 6] = r.i;
    }
    __syncthreads();
    if (tid == 0) {
      ValIdx a{redv[0], redi[0]};
      for (int w = 1; w < (NT + 63) / 64; ++w)
        if (redv[w] > a.v || (redv[w] == a.v && redi[w] < a.i)) a = ValIdx{redv[w], redi[w]};
      if (len == 0) {
        v.score[b] = kNegInf;  // reference: the final alpha is never written
        v.final_c[b] = 0;
      } else {
        v.score[b] = a.v;
        v.final_c[b] = a.i;
      }
    }
  }
}

template <int J, int CMAX>
int launch_vit_j(const Plan& pl, const ViterbiParams& v, int nt, hipStream_t st) {
  const VLds L = vit_lds_layout(pl.C, pl.Kmax, pl.RS, v.ps != nullptr);
  auto k = viterbi_kernel<J, CMAX>;
  hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)L.total);
  if (e != hipSuccess) return e;
  TimedLaunch tl(kKViterbi, st);
  hipLaunchKernelGGL(k, dim3(pl.B), dim3(nt), L.total, st, v);
  return hipGetLastError();
}

// Transition row in registers, C rounded up to a multiple of 8 (CM), for J >= 16.
template <int J>
int launch_vit_cm(const Plan& pl, const ViterbiParams& v, int nt, hipStream_t st) {
  const int cm = (pl.C + 7) / 8 * 8;
  switch (cm) {
    case 8: return launch_vit_j<J, 8>(pl, v, nt, st);
    case 16: return launch_vit_j<J, 16>(pl, v, nt, st);
    case 24: if constexpr (J <= 32) return launch_vit_j<J, 24>(pl, v, nt, st); break;
    case 32: if constexpr (J <= 32) return launch_vit_j<J, 32>(pl, v, nt, st); break;
    case 40: if constexpr (J <= 16) return launch_vit_j<J, 40>(pl, v, nt, st); break;
    case 48: if constexpr (J <= 16) return launch_vit_j<J, 48>(pl, v, nt, st); break;
    case 56: if constexpr (J <= 16) return launch_vit_j<J, 56>(pl, v, nt, st); break;
    case 64: if constexpr (J <= 16) return launch_vit_j<J, 64>(pl, v, nt, st); break;
    default: break;
  }
  return (int)hipErrorInvalidValue;
}

}  // namespace

size_t viterbi_lds_bytes(int C, int Kmax, int RS, int has_ps) { return vit_lds_layout(C, Kmax, RS, has_ps).total; }

// J lanes per label: the largest power of two <= 64 with C*J <= 1024 threads,
// so a sequence's K*C^2 terms per step spread over up to 16 waves.
int launch_viterbi(const Plan& pl, const ViterbiParams& v, hipStream_t s) {
  int J = 64;
  while (J > 1 && pl.C * J > 1024) J >>= 1;
  const int nt = (pl.C * J + 63) / 64 * 64;
  switch (J) {
    case 1: return launch_vit_j<1, 0>(pl, v, nt, s);
    case 2: return launch_vit_j<2, 0>(pl, v, nt, s);
    case 4: return launch_vit_j<4, 0>(pl, v, nt, s);
    case 8: return launch_vit_j<8, 0>(pl, v, nt, s);
    case 16: return launch_vit_cm<16>(pl, v, nt, s);
    case 32: return launch_vit_cm<32>(pl, v, nt, s);
    case 64: return launch_vit_cm<64>(pl, v, nt, s);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace tsm
