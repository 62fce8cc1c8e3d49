// Exact Viterbi (max semiring) with backpointers and on-device backtrace.
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
// registers when it is short enough (CMAX > 0).

#include "tsm_device.hpp"
#include "tsm_internal.hpp"

namespace tsm {
namespace {

struct VLds {
  size_t araw, crng, prng, dbn, trn, red, total;
};

__host__ __device__ inline VLds vit_lds_layout(int C, int Kmax, int RS, int has_ps) {
  VLds L;
  size_t o = 0;
  const size_t ring = sizeof(float) * (size_t)C * RS;
  L.araw = o; o = align16(o + ring);
  L.crng = o; o = align16(o + ring);
  L.prng = o; o = align16(o + (has_ps ? ring : 0));
  L.dbn = o; o = align16(o + sizeof(float) * (size_t)C * (Kmax + 1));
  L.trn = o; o = align16(o + sizeof(float) * (size_t)C * C);
  L.red = o; o = align16(o + sizeof(float) * 64 + sizeof(int) * 64);
  L.total = o;
  return L;
}

template <int J, int CMAX>
__global__ void __launch_bounds__(512) viterbi_kernel(ViterbiParams v) {
  extern __shared__ __align__(16) char smem[];
  const int b = blockIdx.x;
  const int C = v.C, K = v.K, Kmax = v.Kmax, RS = v.RS, T = v.T;
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
    araw[cc * RS] = 0.0f;  // alpha[0, :] = 0
    crng[cc * RS] = cum_b[cc];
    if (has_ps && T > 0) prng[cc * RS] = ps_b[cc];
  }
  __syncthreads();
  float tr_reg[CMAX > 0 ? CMAX : 1];
  if constexpr (CMAX > 0) {
#pragma unroll
    for (int i = 0; i < CMAX; ++i) tr_reg[i] = (i < C) ? trn[c * C + i] : 0.0f;
  }
  const float* dr = dbn + c * (Kmax + 1);
  const float* cr = crng + c * RS;
  const float* pr = prng + c * RS;

  for (int t = 1; t <= len; ++t) {
    const int kcap = (K == 1) ? 1 : min(K - 1, t);
    const int base = t % RS;
    const float cur_cum = cum_b[(size_t)t * C + c];
    const float pe_t = has_pe ? pe_b[(size_t)(t - 1) * C + c] : 0.0f;
    float bv = kMinusInf;
    int bk = 0;
    for (int k = 1 + lj; k <= kcap; k += J) {
      const int slot = wrap_slot(base - k, RS);
      float e1 = (cur_cum - cr[slot]) + dr[k];
      if (has_ps) e1 = e1 + pr[slot];
      if (has_pe) e1 = e1 + pe_t;
      float m = kMinusInf;
      if (v.trows > 0) {
        // duration-dependent transitions: transition[k][c_src][c], from global memory
        const float* tk = v.trans + (size_t)k * C * C + c;
        for (int i = 0; i < C; ++i) m = fmax2(m, araw[i * RS + slot] + (e1 + tk[(size_t)i * C]));
      } else if constexpr (CMAX > 0) {
#pragma unroll
        for (int i = 0; i < CMAX; ++i)
          if (i < C) m = fmax2(m, araw[i * RS + slot] + (e1 + tr_reg[i]));
      } else {
        const float* trow = trn + c * C;
        for (int i = 0; i < C; ++i) m = fmax2(m, araw[i * RS + slot] + (e1 + trow[i]));
      }
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
        const float x = araw[i * RS + slot] + (e1 + (v.trows > 0 ? tk[(size_t)i * C] : trn[c * C + i]));
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
      araw[c * RS + base] = best.v;
      crng[c * RS + base] = cur_cum;
      if (has_ps && t < T) prng[c * RS + base] = ps_b[(size_t)t * C + c];
    }
    __syncthreads();
  }
  // ---- score = max over labels of alpha[len]; first maximising label ----
  {
    const int slot = len % RS;
    float mv = kMinusInf;
    int mi = 0x7fffffff;
    for (int cc = tid; cc < C; cc += NT) {
      const float x = araw[cc * RS + slot];
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

// One thread per sequence walks the backpointers from (len, final label).
__global__ void backtrace_kernel(ViterbiParams v) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= v.B) return;
  const int C = v.C, T = v.T;
  int64_t L64 = v.lengths[b];
  const int len = (int)(L64 < 0 ? 0 : (L64 > T ? T : L64));
  int t = len, c = v.final_c[b], n = 0;
  int32_t* out = v.segs + (size_t)b * T * 4;
  while (t > 0 && n < T) {
    const int32_t w = v.bp[((size_t)b * (T + 1) + t) * C + c];
    const int k = w >> 16, cp = w & 0xffff;
    if (k <= 0 || k > t || cp >= C) break;
    out[4 * n + 0] = t - k;
    out[4 * n + 1] = t - 1;
    out[4 * n + 2] = c;
    out[4 * n + 3] = cp;
    ++n;
    t -= k;
    c = cp;
  }
  v.seg_count[b] = n;
}

// Backtrace with the backpointers staged in LDS, one workgroup per sequence.
// Rows [q*TCH, (q+1)*TCH) of bp (all labels) form chunk q; TCH > Kmax, so every
// read of the walk lies in the current chunk or the one below, and while wave 0
// walks chunk q the other waves load chunk q-1 into the second buffer
// (coalesced rows), so the walk's dependent reads hit LDS instead of HBM.  The
// segments of a chunk are buffered in LDS and written out by the whole
// workgroup.
// bp[t,c] = (k << 16 | c_prev): segment [t-k, t-1] of label c, then (t-k, c_prev)
// (the exact kernel's format; the factorised scan's is converted first, see
// fact_to_exact_kernel).  Final label: final_c[b] (FIN = false) or the first
// maximiser of fin[b, :] (FIN = true).
template <bool FIN>
__global__ void __launch_bounds__(256) backtrace_lds_kernel(const int32_t* bp, const float* fin,
                                                            const int32_t* final_c, const int64_t* lengths, int B,
                                                            int T, int C, int TCH, int32_t* seg_count, int32_t* segs) {
  extern __shared__ __align__(16) int32_t sbuf[];  // 2 bp chunks of TCH*C, then TCH segments of 4
  __shared__ int next_q, chunk_segs;
  const int b = blockIdx.x;
  const int tid = threadIdx.x, NT = blockDim.x;
  int64_t L64 = lengths[b];
  const int len = (int)(L64 < 0 ? 0 : (L64 > T ? T : L64));
  if (len == 0) {
    if (tid == 0) seg_count[b] = 0;
    return;
  }
  const int32_t* bpb = bp + (size_t)b * (T + 1) * C;
  int32_t* out = segs + (size_t)b * T * 4;
  int4* sseg = reinterpret_cast<int4*>(sbuf + (size_t)2 * TCH * C);
  // chunk rows to LDS, four loads in flight per thread
  auto load = [&](int q, int32_t* buf, int first, int stride) {
    const int lo = q * TCH, n = min(TCH, T + 1 - lo) * C;
    const int32_t* src = bpb + (size_t)lo * C;
    int i = first;
    for (; i + 3 * stride < n; i += 4 * stride) {
      const int32_t a0 = src[i], a1 = src[i + stride], a2 = src[i + 2 * stride], a3 = src[i + 3 * stride];
      buf[i] = a0;
      buf[i + stride] = a1;
      buf[i + 2 * stride] = a2;
      buf[i + 3 * stride] = a3;
    }
    for (; i < n; i += stride) buf[i] = src[i];
  };
  int q = len / TCH;
  load(q, sbuf, tid, NT);
  // walk state: position t, label c
  int t = len, c = 0;
  if (tid == 0) {
    if (FIN) {
      float best = fin[(size_t)b * C];
      for (int cc = 1; cc < C; ++cc) {
        const float x = fin[(size_t)b * C + cc];
        if (x > best) {
          best = x;
          c = cc;
        }
      }
    } else {
      c = final_c[b];
    }
  }
  c = __builtin_amdgcn_readfirstlane(c);  // wave 0's walk state is wave-uniform (others ignore it)
  __syncthreads();
  int cur = 0, nbase = 0;
  // wave index as a provably uniform value, so wave 0's walk compiles to scalar code
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  for (;;) {
    const int lo = q * TCH;
    const int32_t* buf = sbuf + (size_t)cur * TCH * C;
    if (wave != 0) {
      // waves 1.. prefetch the next chunk; wave 0 is left to the walk (a divergent
      // wave would run the loads and the walk one after the other)
      if (q > 0) load(q - 1, sbuf + (size_t)(cur ^ 1) * TCH * C, tid - 64, NT - 64);
    } else {
      // wave 0 walks, all lanes together on wave-uniform values (broadcast LDS
      // reads, scalar control flow); the chunk's segments go to LDS and the
      // workgroup writes them out below
      int m = 0;
      while (t > 0 && t >= lo) {
        const int32_t w = __builtin_amdgcn_readfirstlane(buf[(t - lo) * C + c]);
        const int k = w >> 16, cp = w & 0xffff;
        if (k <= 0 || k > t || cp >= C) {  // no segment ends here (or not a label): stop
          t = 0;
          break;
        }
        if (tid == 0) sseg[m] = make_int4(t - k, t - 1, c, cp);
        ++m;
        t -= k;
        c = cp;
      }
      if (tid == 0) {
        chunk_segs = m;
        next_q = (t > 0 && q > 0) ? q - 1 : -1;
      }
    }
    __syncthreads();
    const int m = chunk_segs, nq = next_q;
    const int32_t* sv = reinterpret_cast<const int32_t*>(sseg);
    for (int i = tid; i < 4 * m; i += NT) out[4 * (size_t)nbase + i] = sv[i];
    nbase += m;
    if (nq < 0) break;
    q = nq;
    cur ^= 1;
    __syncthreads();  // the segment buffer and next_q are read by all before thread 0 rewrites them
  }
  if (tid == 0) seg_count[b] = nbase;
}

// Factorised backpointers (k* at (t,c) for a segment ending at t, best source at
// (s,c) for a segment starting at s) to the exact format (k << 16 | c_prev) of
// the segment ending at t, so the backtrace needs one dependent read per
// segment instead of two.  0 where no segment ends (t = 0, t > len, bad k).
__global__ void fact_to_exact_kernel(const int32_t* bp, const int64_t* lengths, int B, int T, int C, int32_t* out) {
  const size_t n = (size_t)B * (T + 1) * C;
  for (size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (size_t)gridDim.x * blockDim.x) {
    const int c = (int)(idx % C);
    const int t = (int)((idx / C) % (T + 1));
    const int b = (int)(idx / ((size_t)C * (T + 1)));
    int64_t L64 = lengths[b];
    const int len = (int)(L64 < 0 ? 0 : (L64 > T ? T : L64));
    int32_t v = 0;
    if (t >= 1 && t <= len) {
      const int k = bp[idx] >> 16;
      if (k >= 1 && k <= t) v = (k << 16) | (bp[idx - (size_t)k * C] & 0xffff);
    }
    out[idx] = v;
  }
}

// LDS bytes of backtrace_lds_kernel: two bp chunks and a chunk's segments.
size_t backtrace_lds_bytes(int tch, int C) { return (size_t)tch * C * 8 + (size_t)tch * 16; }

// Rows per chunk of backtrace_lds_kernel (0: chunks of Kmax+1 rows do not fit in LDS).
int backtrace_chunk_rows(int C, int Kmax, int max_lds) {
  const size_t cap = (size_t)max_lds - 64;
  int tch = 256;
  while (backtrace_lds_bytes(tch, C) > cap && tch > 1) tch >>= 1;
  if (tch <= Kmax) tch = Kmax + 1;
  return backtrace_lds_bytes(tch, C) <= cap ? tch : 0;
}

int max_lds_bytes() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) {
    (void)hipGetLastError();
    return 64 * 1024;
  }
  return v;
}

template <bool FACT>
int launch_backtrace_lds(int tch, const int32_t* bp, const float* fin, const int32_t* final_c, const int64_t* lengths,
                         int B, int T, int C, int32_t* seg_count, int32_t* segs, hipStream_t st) {
  auto k = backtrace_lds_kernel<FACT>;
  const size_t lds = backtrace_lds_bytes(tch, C);
  hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  TimedLaunch tl(kKBacktrace, st);
  hipLaunchKernelGGL(k, dim3(B), dim3(256), lds, st, bp, fin, final_c, lengths, B, T, C, tch, seg_count, segs);
  return hipGetLastError();
}

template <int J, int CMAX>
int launch_vit_j(const Plan& pl, const ViterbiParams& v, int with_tb, hipStream_t st) {
  const VLds L = vit_lds_layout(pl.C, pl.Kmax, pl.RS, v.ps != nullptr);
  auto k = viterbi_kernel<J, CMAX>;
  hipError_t e = hipFuncSetAttribute((const void*)k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)L.total);
  if (e != hipSuccess) return e;
  {
    TimedLaunch tl(kKViterbi, st);
    hipLaunchKernelGGL(k, dim3(pl.B), dim3(pl.NT), L.total, st, v);
  }
  if (with_tb) {
    const int tch = backtrace_chunk_rows(pl.C, pl.Kmax, max_lds_bytes());
    if (tch > 0)
      return launch_backtrace_lds<false>(tch, v.bp, nullptr, v.final_c, v.lengths, pl.B, pl.T, pl.C, v.seg_count,
                                         v.segs, st);
    TimedLaunch tl(kKBacktrace, st);
    hipLaunchKernelGGL(backtrace_kernel, dim3((pl.B + 63) / 64), dim3(64), 0, st, v);
  }
  return hipGetLastError();
}

// Backtrace of the factorised Viterbi (one thread per sequence).  bp[t,c] holds
// (k << 16 | c') with k the best duration of a segment of label c ending at t
// and c' the best source label of a segment of label c starting at t, so the
// previous label of the segment [t-k, t-1] is bp[t-k, c] & 0xffff.  The final
// label is the first maximiser of the normalised final row fin[b, :].
__global__ void backtrace_fact_kernel(const int32_t* bp, const float* fin, const int64_t* lengths, int B, int T,
                                      int C, int32_t* seg_count, int32_t* segs) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= B) return;
  int64_t L64 = lengths[b];
  const int len = (int)(L64 < 0 ? 0 : (L64 > T ? T : L64));
  int c = 0;
  float best = fin[(size_t)b * C];
  for (int cc = 1; cc < C; ++cc) {
    const float x = fin[(size_t)b * C + cc];
    if (x > best) {
      best = x;
      c = cc;
    }
  }
  int t = len, n = 0;
  int32_t* out = segs + (size_t)b * T * 4;
  const int32_t* bpb = bp + (size_t)b * (T + 1) * C;
  while (t > 0 && n < T) {
    const int k = bpb[(size_t)t * C + c] >> 16;
    if (k <= 0 || k > t) break;
    const int s = t - k;
    const int cp = bpb[(size_t)s * C + c] & 0xffff;
    if (cp >= C) break;
    out[4 * n + 0] = s;
    out[4 * n + 1] = t - 1;
    out[4 * n + 2] = c;
    out[4 * n + 3] = cp;
    ++n;
    t = s;
    c = cp;
  }
  seg_count[b] = n;
}

}  // namespace

int launch_backtrace_fact(const Plan& pl, const int32_t* bp, int32_t* bp_exact, const float* fin,
                          const int64_t* lengths, int32_t* seg_count, int32_t* segs, hipStream_t s) {
  const int tch = backtrace_chunk_rows(pl.C, pl.Kmax, max_lds_bytes());
  if (tch > 0) {
    const size_t n = (size_t)pl.B * (pl.T + 1) * pl.C;
    int g = (int)((n + 255) / 256);
    if (g > 8192) g = 8192;
    {
      TimedLaunch tl(kKBacktrace, s);
      hipLaunchKernelGGL(fact_to_exact_kernel, dim3(g), dim3(256), 0, s, bp, lengths, pl.B, pl.T, pl.C, bp_exact);
    }
    return launch_backtrace_lds<true>(tch, bp_exact, fin, nullptr, lengths, pl.B, pl.T, pl.C, seg_count, segs, s);
  }
  TimedLaunch tl(kKBacktrace, s);
  hipLaunchKernelGGL(backtrace_fact_kernel, dim3((pl.B + 63) / 64), dim3(64), 0, s, bp, fin, lengths, pl.B, pl.T,
                     pl.C, seg_count, segs);
  return hipGetLastError();
}

size_t viterbi_lds_bytes(int C, int Kmax, int RS, int has_ps) { return vit_lds_layout(C, Kmax, RS, has_ps).total; }

int launch_viterbi(const Plan& pl, const ViterbiParams& v, int with_traceback, hipStream_t s) {
  switch (pl.J) {
    case 1: return launch_vit_j<1, 0>(pl, v, with_traceback, s);
    case 2: return launch_vit_j<2, 0>(pl, v, with_traceback, s);
    case 4: return launch_vit_j<4, 0>(pl, v, with_traceback, s);
    case 8: return launch_vit_j<8, 64>(pl, v, with_traceback, s);
    case 16: return launch_vit_j<16, 32>(pl, v, with_traceback, s);
    case 32: return launch_vit_j<32, 16>(pl, v, with_traceback, s);
    case 64: return launch_vit_j<64, 8>(pl, v, with_traceback, s);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace tsm
