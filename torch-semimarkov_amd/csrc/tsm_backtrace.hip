// Chunked, speculative Viterbi backtrace (reference: nn.py:444-531
// `_traceback_single`, one Python loop per sequence).
//
// bp[b,t,c] = (k << 16 | c_prev): the best segment of label c ending at t is
// [t-k, t-1], and the node before it is (t-k, c_prev); 0 where no segment ends.
// The path of sequence b is the chain of nodes from (len, c_final) down to
// position 0.  One walk is a chain of dependent reads, so a long sequence is
// cut into chunks of Lc upper-node positions (lo_j, hi_j] and all chunks walk
// at once:
//   * the top chunk (it contains len) walks exactly from (len, c_final);
//   * every chunk below starts D positions above its range at label 0 and
//     records the segments whose upper node lies in (lo_j, hi_j], then stops at
//     its exit node (the first node at or below lo_j).
// Two walks that share a node coincide from there on, and backpointer chains
// from different starts merge after a few segments (survivor-path merging),
// so chunk j's record is the true path from the true entry node -- the exit
// node of chunk j+1, once that chunk is right -- whenever the record contains
// that node.  A parallel pass finds the entry node in each record (binary
// search: records are in decreasing position order); a per-sequence pass then
// goes from the top down, re-searches where the chunk above changed, re-walks
// exactly from the true entry node every chunk whose record misses it (so the
// result never depends on the speculation), and turns the counts into output
// offsets; a last parallel pass copies each chunk's valid records into place.
// Chunks are at least Kmax+1 long, so an entry node always falls inside the
// chunk below.
//
// Walks stage the backpointer rows in LDS, TCH > Kmax rows at a time (every
// next node then lies in the current stage or the one below): waves 1.. load
// the next stage while wave 0 walks on wave-uniform (scalar) values.  When two
// stages do not fit in LDS (TCH = 0) wave 0 reads the rows from global memory.

#include <stdlib.h>
#include <string.h>

#include <algorithm>

#include "tsm_device.hpp"
#include "tsm_internal.hpp"

namespace tsm {
namespace {

constexpr int kBtThreads = 256;

struct BtParams {
  const int32_t* bp;       // (B, T+1, C), exact format
  const float* fin;        // (B, C) final row: path starts at its first maximiser, or null
  const int32_t* final_c;  // (B) final label (used when fin is null)
  const int64_t* lengths;
  int B, T, C, Kmax;
  int P, Lc, D, TCH;
  int4* lists;             // (B*P, Lc) records (start, end, label, previous label)
  int* nseg;               // (B*P)
  int* first;              // (B*P) first valid record, -1: entry node not found
  int* off;                // (B*P) output offset of the first valid record
  int2* exitn;             // (B*P) exit node (t, c); t = 0 when the chain ended
  int32_t* seg_count;      // (B)
  int32_t* segs;           // (B, T, 4)
};

__device__ __forceinline__ int bt_len(const BtParams& p, int b) {
  int64_t L = p.lengths[b];
  return (int)(L < 0 ? 0 : (L > p.T ? p.T : L));
}

__device__ __forceinline__ int bt_nch(const BtParams& p, int len) { return len == 0 ? 0 : (len + p.Lc - 1) / p.Lc; }

// Walk of sequence b from node (t0, c0) down to the first node at or below
// lo, recording the segments whose upper node is <= hi into rec[0..).  All
// threads of the block call it with the same arguments; afterwards sh[0] holds
// the record count and sh[1], sh[2] the exit node.
template <bool STAGED>
__device__ void bt_walk(const BtParams& p, int b, int lo, int hi, int t0, int c0, int4* rec, int32_t* sbuf,
                        int* sh) {
  const int C = p.C, TCH = p.TCH, tid = threadIdx.x;
  const int32_t* bpb = p.bp + (size_t)b * (p.T + 1) * C;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  int t = __builtin_amdgcn_readfirstlane(t0), c = __builtin_amdgcn_readfirstlane(c0), n = 0;
  // one step of the walk on wave-uniform values; false when the chain ends
  auto step = [&](int32_t w) -> bool {
    const int k = w >> 16, cp = w & 0xffff;
    if (k <= 0 || k > t || cp >= C) return false;
    if (t <= hi && n < p.Lc) {
      if (tid == 0) rec[n] = make_int4(t - k, t - 1, c, cp);
      ++n;
    }
    t -= k;
    c = cp;
    return true;
  };
  if constexpr (!STAGED) {
    if (wave == 0) {
      while (t > lo) {
        if (!step(__builtin_amdgcn_readfirstlane(bpb[(size_t)t * C + c]))) {
          t = 0;
          c = 0;
          break;
        }
      }
      if (tid == 0) {
        sh[0] = n;
        sh[1] = t;
        sh[2] = c;
      }
    }
    __syncthreads();
    return;
  } else {
    __shared__ int next_q;
    // rows of stage q to LDS, eight loads in flight per thread
    auto load = [&](int q, int32_t* buf, int first, int stride) {
      const int r0 = q * TCH, cnt = min(TCH, p.T + 1 - r0) * C;
      const int32_t* src = bpb + (size_t)r0 * C;
      int i = first;
      for (; i + 7 * stride < cnt; i += 8 * stride) {
        int32_t a[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) a[u] = src[i + u * stride];
#pragma unroll
        for (int u = 0; u < 8; ++u) buf[i + u * stride] = a[u];
      }
      for (; i < cnt; i += stride) buf[i] = src[i];
    };
    const int qmin = (lo + 1) / TCH;
    int q = t / TCH, cur = 0;
    load(q, sbuf, tid, blockDim.x);
    __syncthreads();
    for (;;) {
      const int r0 = q * TCH;
      const int32_t* buf = sbuf + (size_t)cur * TCH * C;
      if (wave != 0) {
        if (q > qmin) load(q - 1, sbuf + (size_t)(cur ^ 1) * TCH * C, tid - 64, blockDim.x - 64);
      } else {
        while (t > lo && t >= r0) {
          if (!step(__builtin_amdgcn_readfirstlane(buf[(t - r0) * C + c]))) {
            t = 0;
            c = 0;
            break;
          }
        }
        if (tid == 0) next_q = (t > lo && q > qmin) ? q - 1 : -1;
      }
      __syncthreads();
      const int nq = next_q;
      if (nq < 0) break;
      q = nq;
      cur ^= 1;
      __syncthreads();  // next_q is read by all before thread 0 rewrites it
    }
    if (tid == 0) {
      sh[0] = n;
      sh[1] = t;
      sh[2] = c;
    }
    __syncthreads();
  }
}

// Parallel pass: one block per (sequence, chunk).
template <bool STAGED>
__global__ void __launch_bounds__(kBtThreads) bt_chunk_kernel(BtParams p) {
  extern __shared__ __align__(16) int32_t sbuf[];
  __shared__ int sh[3];
  const int b = blockIdx.x / p.P, j = blockIdx.x % p.P, item = blockIdx.x;
  const int len = bt_len(p, b), nch = bt_nch(p, len);
  if (j >= nch) {
    if (threadIdx.x == 0) {
      p.nseg[item] = 0;
      p.first[item] = 0;
      p.exitn[item] = make_int2(0, 0);
    }
    return;
  }
  const int lo = j * p.Lc, hi = min(lo + p.Lc, len);
  int t0, c0 = 0;
  if (j == nch - 1) {
    t0 = len;
    if (p.fin != nullptr) {
      float best = p.fin[(size_t)b * p.C];
      for (int cc = 1; cc < p.C; ++cc) {
        const float x = p.fin[(size_t)b * p.C + cc];
        if (x > best) {
          best = x;
          c0 = cc;
        }
      }
    } else {
      c0 = p.final_c[b];
    }
  } else {
    t0 = min(hi + p.D, len);
  }
  bt_walk<STAGED>(p, b, lo, hi, t0, c0, p.lists + (size_t)item * p.Lc, sbuf, sh);
  if (threadIdx.x == 0) {
    p.nseg[item] = sh[0];
    p.exitn[item] = make_int2(sh[1], sh[2]);
    p.first[item] = 0;
  }
}

// Index of the record whose upper node is (E.x, E.y) in rec[0..n), or -1.
__device__ int bt_find(const int4* rec, int n, int2 E) {
  int a = 0, z = n - 1;
  while (a <= z) {
    const int m = (a + z) >> 1;
    const int4 r = rec[m];
    const int up = r.y + 1;
    if (up == E.x) return r.z == E.y ? m : -1;
    if (up > E.x) a = m + 1;
    else z = m - 1;
  }
  return -1;
}

// Parallel verification: chunk j against the (possibly speculative) exit node
// of chunk j+1.
__global__ void bt_verify_kernel(BtParams p) {
  const int item = blockIdx.x * blockDim.x + threadIdx.x;
  if (item >= p.B * p.P) return;
  const int b = item / p.P, j = item % p.P;
  const int nch = bt_nch(p, bt_len(p, b));
  if (j >= nch - 1) return;  // top chunk (exact) or no chunk
  const int2 E = p.exitn[item + 1];
  const int n = p.nseg[item];
  p.first[item] = E.x <= 0 ? n : bt_find(p.lists + (size_t)item * p.Lc, n, E);
}

// Per-sequence pass, top chunk down: re-verify below a re-walked chunk, re-walk
// exactly where the entry node is missing, then output offsets.
template <bool STAGED>
__global__ void __launch_bounds__(kBtThreads) bt_fixup_kernel(BtParams p) {
  extern __shared__ __align__(16) int32_t sbuf[];
  __shared__ int s_first[kBtMaxChunks], s_nseg[kBtMaxChunks];
  __shared__ int2 s_exit[kBtMaxChunks];
  __shared__ int sh[3];
  __shared__ int s_redo, s_changed;
  __shared__ int2 s_E;
  const int b = blockIdx.x, tid = threadIdx.x;
  const int len = bt_len(p, b), nch = bt_nch(p, len);
  if (nch == 0) {
    if (tid == 0) p.seg_count[b] = 0;
    return;
  }
  const size_t base = (size_t)b * p.P;
  for (int j = tid; j < nch; j += blockDim.x) {
    s_first[j] = p.first[base + j];
    s_nseg[j] = p.nseg[base + j];
    s_exit[j] = p.exitn[base + j];
  }
  if (tid == 0) {
    s_first[nch - 1] = 0;
    s_changed = 0;
  }
  __syncthreads();
  for (int j = nch - 2; j >= 0; --j) {
    if (tid == 0) {
      const int2 E = s_exit[j + 1];
      int f = s_first[j];
      if (E.x <= 0) {
        f = s_nseg[j];  // the chain ended above: nothing below is on the path
        s_exit[j] = make_int2(0, 0);
      } else if (s_changed) {
        f = bt_find(p.lists + (base + j) * p.Lc, s_nseg[j], E);
      }
      s_first[j] = f;
      s_redo = f < 0;
      s_E = E;
    }
    __syncthreads();
    if (s_redo) {
      const int lo = j * p.Lc, hi = min(lo + p.Lc, len);
      const int2 E = s_E;
      bt_walk<STAGED>(p, b, lo, hi, E.x, E.y, p.lists + (base + j) * p.Lc, sbuf, sh);
      if (tid == 0) {
        s_nseg[j] = sh[0];
        s_exit[j] = make_int2(sh[1], sh[2]);
        s_first[j] = 0;
        s_changed = 1;
      }
    } else if (tid == 0) {
      s_changed = 0;
    }
    __syncthreads();
  }
  if (tid == 0) {
    int total = 0;
    for (int j = nch - 1; j >= 0; --j) {
      p.off[base + j] = total;
      total += s_nseg[j] - s_first[j];
    }
    p.seg_count[b] = total;
  }
  for (int j = tid; j < nch; j += blockDim.x) {
    p.first[base + j] = s_first[j];
    p.nseg[base + j] = s_nseg[j];
  }
}

// Valid records of every chunk to their place in the output.
__global__ void __launch_bounds__(kBtThreads) bt_copy_kernel(BtParams p) {
  const int item = blockIdx.x, b = item / p.P, j = item % p.P;
  if (j >= bt_nch(p, bt_len(p, b))) return;
  const int f = p.first[item], n = p.nseg[item] - f, o = p.off[item];
  const int4* src = p.lists + (size_t)item * p.Lc + f;
  int32_t* dst = p.segs + ((size_t)b * p.T + o) * 4;
  for (int i = threadIdx.x; i < n; i += blockDim.x) {
    if (o + i >= p.T) break;
    const int4 r = src[i];
    dst[4 * i + 0] = r.x;
    dst[4 * i + 1] = r.y;
    dst[4 * i + 2] = r.z;
    dst[4 * i + 3] = r.w;
  }
}

// Factorised backpointers (k* at (t,c) for a segment ending at t, best source
// at (s,c) for a segment starting at s) to the exact format (k << 16 | c_prev)
// of the segment ending at t, so a walk needs one dependent read per segment
// instead of two.  0 where no segment ends (t = 0, t > len, bad k).
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

int device_max_lds() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || v <= 0) {
    (void)hipGetLastError();
    return 64 * 1024;
  }
  return v;
}

int device_cus() {
  int dev = 0, v = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) {
    (void)hipGetLastError();
    return 256;
  }
  return v;
}

template <bool STAGED>
int launch_bt(const BtParams& p, hipStream_t st) {
  const size_t lds = STAGED ? (size_t)2 * p.TCH * p.C * sizeof(int32_t) : 0;
  auto kc = bt_chunk_kernel<STAGED>;
  auto kf = bt_fixup_kernel<STAGED>;
  hipError_t e = hipFuncSetAttribute((const void*)kc, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  e = hipFuncSetAttribute((const void*)kf, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
  if (e != hipSuccess) return e;
  const int items = p.B * p.P;
  hipLaunchKernelGGL(kc, dim3(items), dim3(kBtThreads), lds, st, p);
  hipLaunchKernelGGL(bt_verify_kernel, dim3((items + 255) / 256), dim3(256), 0, st, p);
  hipLaunchKernelGGL(kf, dim3(p.B), dim3(kBtThreads), lds, st, p);
  hipLaunchKernelGGL(bt_copy_kernel, dim3(items), dim3(kBtThreads), 0, st, p);
  return hipGetLastError();
}

}  // namespace

BtPlan backtrace_plan(int B, int T, int C, int Kmax) {
  BtPlan bp;
  // two stages of TCH > Kmax rows in LDS (the fixup kernel's static arrays aside)
  const size_t cap = (size_t)device_max_lds() - 16 * 1024;
  int tch = 1024;
  while (tch > 1 && (size_t)8 * tch * C > cap) tch >>= 1;
  if (tch <= Kmax) tch = Kmax + 1;
  bp.TCH = ((size_t)8 * tch * C <= cap) ? tch : 0;
  // TSM_BACKTRACE_PATH=global: walks read the rows from global memory (tests)
  const char* env = getenv("TSM_BACKTRACE_PATH");
  if (env != nullptr && strcmp(env, "global") == 0) bp.TCH = 0;
  // about one chunk per CU, chunks of at least max(4 (Kmax+1), 1024) positions; when that
  // leaves most CUs idle, the walks' length is the time (a chunk walks D positions into its
  // range and then its own Lc), so chunks go down to D/2 (at B=4, T=1000, K=100: walks of
  // about 400 positions instead of one of 1000)
  bp.D = 2 * (Kmax + 1) + 64;
  const int64_t cus = device_cus();
  int64_t min_lc = std::max<int64_t>(4 * ((int64_t)Kmax + 1), 1024);
  if ((int64_t)B * std::max<int64_t>(1, (int64_t)T / min_lc) < cus) min_lc = std::max<int64_t>(bp.D / 2, 64);
  int64_t P = (cus + (int64_t)B - 1) / B;
  P = std::min<int64_t>(P, std::max<int64_t>(1, (int64_t)T / min_lc));
  P = std::max<int64_t>(1, std::min<int64_t>(P, kBtMaxChunks));
  bp.P = (int)P;
  bp.Lc = (int)(((int64_t)T + P - 1) / P);
  return bp;
}

size_t backtrace_ws_bytes(const BtPlan& bp, int B) {
  const size_t items = (size_t)B * bp.P;
  return items * bp.Lc * sizeof(int4) + items * (3 * sizeof(int) + sizeof(int2)) + 4 * 256;
}

int launch_backtrace(const BtPlan& bpl, const int32_t* bp, const float* fin, const int32_t* final_c,
                     const int64_t* lengths, int B, int T, int C, int Kmax, void* ws, int32_t* seg_count,
                     int32_t* segs, hipStream_t st) {
  BtParams p{};
  p.bp = bp;
  p.fin = fin;
  p.final_c = final_c;
  p.lengths = lengths;
  p.B = B;
  p.T = T;
  p.C = C;
  p.Kmax = Kmax;
  p.P = bpl.P;
  p.Lc = bpl.Lc;
  p.D = bpl.D;
  p.TCH = bpl.TCH;
  const size_t items = (size_t)B * bpl.P;
  char* w = static_cast<char*>(ws);
  auto take = [&](size_t bytes) {
    char* r = w;
    w += (bytes + 255) & ~size_t(255);
    return r;
  };
  p.lists = reinterpret_cast<int4*>(take(items * bpl.Lc * sizeof(int4)));
  p.nseg = reinterpret_cast<int*>(take(items * sizeof(int)));
  p.first = reinterpret_cast<int*>(take(items * sizeof(int)));
  p.off = reinterpret_cast<int*>(take(items * sizeof(int)));
  p.exitn = reinterpret_cast<int2*>(take(items * sizeof(int2)));
  p.seg_count = seg_count;
  p.segs = segs;
  TimedLaunch tl(kKBacktrace, st);
  return bpl.TCH > 0 ? launch_bt<true>(p, st) : launch_bt<false>(p, st);
}

// Score terms of the segment rows of a traceback, one thread per row: the row
// (start, end, label, previous label) becomes (start, end, label, content,
// duration bias, transition) in fp64, content the fp32 difference of two
// cumulative scores (nn.py:532-555).  Indices are clamped into their tensors.
__global__ void segment_terms_kernel(const float* cum, const float* tr, const float* db, const int32_t* seg_count,
                                     const int32_t* segs, int T, int C, int K, double* out) {
  const int b = blockIdx.y;
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= T || i >= seg_count[b]) return;
  const int4 r = reinterpret_cast<const int4*>(segs)[(size_t)b * T + i];
  auto clampi = [](int v, int lo, int hi) { return v < lo ? lo : (v > hi ? hi : v); };
  const int s = clampi(r.x, 0, T - 1), e = clampi(r.y, 0, T - 1);
  const int l = clampi(r.z, 0, C - 1), pv = clampi(r.w, 0, C - 1);
  const float* cb = cum + (size_t)b * (T + 1) * C;
  const float content = cb[(size_t)(e + 1) * C + l] - cb[(size_t)s * C + l];
  const int dur = e - s + 1;
  const int di = clampi(dur, 0, K - 1);
  double* o = out + ((size_t)b * T + i) * 6;
  o[0] = (double)r.x;
  o[1] = (double)r.y;
  o[2] = (double)r.z;
  o[3] = (double)content;
  o[4] = (double)db[(size_t)di * C + l];
  o[5] = (double)tr[(size_t)pv * C + l];
}

int launch_segment_terms(const float* cum, const float* tr, const float* db, const int32_t* seg_count,
                         const int32_t* segs, int B, int T, int C, int K, double* out, hipStream_t st) {
  if (B == 0 || T == 0) return hipSuccess;
  TimedLaunch tl(kKBacktrace, st);
  hipLaunchKernelGGL(segment_terms_kernel, dim3((T + 255) / 256, B), dim3(256), 0, st, cum, tr, db, seg_count, segs, T,
                     C, K, out);
  return hipGetLastError();
}

int launch_fact_to_exact(const int32_t* bp, const int64_t* lengths, int B, int T, int C, int32_t* out,
                         hipStream_t st) {
  const size_t n = (size_t)B * (T + 1) * C;
  int g = (int)((n + 255) / 256);
  if (g > 8192) g = 8192;
  TimedLaunch tl(kKBacktrace, st);
  hipLaunchKernelGGL(fact_to_exact_kernel, dim3(g), dim3(256), 0, st, bp, lengths, B, T, C, out);
  return hipGetLastError();
}

}  // namespace tsm
