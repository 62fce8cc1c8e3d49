// Bookkeeping kernels of the bounded-memory (checkpointed) backward.
//
// The forward keeps, per sequence b and window w >= 1 (windows of `Wlen`
// positions, whole chunks of the forward's plan), the state the chunk ending at
// the window start recorded -- the Kmax ring entries of positions a_w, a_w-1, ...
// in the ring format of the register-resident scan -- and the alpha-hat row at
// a_w, with levels in the global frame.  The backward then runs each window as
// a problem of its own, top window first: the forward over the window from its
// start state (recomputing alpha-hat for Wlen positions), then the fused
// backward from the state that the window above recorded at its position 0.
// These kernels compute the per-window lengths and flags, move the records
// into the global frame, and add the end sums that a window's segments leave
// in the window above.  Reference counterpart: the checkpointed recomputation
// of streaming/pytorch_reference.py:380-423 (alpha recomputed per segment from
// ring checkpoints), here per window of whole chunks.
#include <algorithm>

#include "tsm_internal.hpp"

namespace tsm {
namespace {

__device__ inline int wlen_of(const int64_t* lengths, int b, int T) {
  int64_t L = lengths[b];
  if (L < 0) L = 0;
  if (L > T) L = T;
  return (int)L;
}

// Per (w, b), index w*B + b: window length len_w = clamp(len_b - a_w, 0, T_w),
// whether the window starts from a recorded forward state (w >= 1 and the
// sequence reaches into it) and whether it ends on one of the window above (the
// sequence goes beyond it).
__global__ void window_setup_kernel(const int64_t* lengths, int B, int T, int Wlen, int nw, int64_t* lenw, int* okf,
                                    int* okb) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= B * nw) return;
  const int w = i / B, b = i % B;
  const int len = wlen_of(lengths, b, T);
  const int a = w * Wlen, Tw = min(Wlen, T - a);
  lenw[i] = (int64_t)max(0, min(len - a, Tw));
  okf[i] = (w >= 1 && len > a) ? 1 : 0;
  okb[i] = (len > a + Tw) ? 1 : 0;
}

// Records of the forward's chunks ending at window starts -> global frame.
// Block (w - 1, b): chunk it = b*P + w*Wc - 1 ended at a_w; its ring entries
// copy over, its levels (and the alpha-hat row's level recorded at a_w) take its
// verified offset.  Checkpoint layout (window, sequence, ...).
__global__ void ck_extract_kernel(const float* st_end, const double* lv_end, const double* offs, int B, int P, int Wc,
                                  int Kmax, int C, float* ck_st, double* ck_lv, double* ck_al) {
  const int w = blockIdx.x + 1, b = blockIdx.y;
  const size_t it = (size_t)b * P + (size_t)w * Wc - 1;
  const size_t o = (size_t)w * B + b;
  const double off = offs[it];
  for (int i = threadIdx.x; i < Kmax * C; i += blockDim.x) ck_st[o * Kmax * C + i] = st_end[it * Kmax * C + i];
  for (int i = threadIdx.x; i < Kmax; i += blockDim.x) ck_lv[o * Kmax + i] = lv_end[it * Kmax + i] + off;
  if (threadIdx.x == 0) ck_al[o] += off;
}

// Row 0 of each sequence's alpha-hat table of a window (the forward writes rows
// 1..T_w) from the window's checkpoints (ck_ah (B, C), ck_al (B,)), for the
// sequences that start from a recorded state.  Block b.
__global__ void window_row0_kernel(const float* ck_ah, const double* ck_al, const int* okf, int Tw, int C, float* ah,
                                   double* al) {
  const int b = blockIdx.x;
  if (okf[b] == 0) return;
  for (int c = threadIdx.x; c < C; c += blockDim.x) ah[(size_t)b * (Tw + 1) * C + c] = ck_ah[(size_t)b * C + c];
  if (threadIdx.x == 0) al[(size_t)b * (Tw + 1)] = ck_al[b];
}

// The state chunk 0 of a window's backward recorded at position 0, in its frame,
// -> global frame (its verified offset).  Block b.
__global__ void window_state_fix_kernel(double* lv, const double* offs, int P, int Kmax) {
  const int b = blockIdx.x;
  for (int i = threadIdx.x; i < Kmax; i += blockDim.x) lv[(size_t)b * Kmax + i] += offs[(size_t)b * P];
}

// End sums of segments starting in the window and ending in the window above
// (positions len_w + 1 .. len_w + Kmax - 1 of the window, the first rows of the
// one above), added into the cum / proj_end gradients with grad_output and the
// chunk factors: the top chunk jl sent them to thalo, the chunk below it (when
// jl >= 1) kept them in its halo rows.  gcum_e / gpe_e point at row a_w + T_w
// of sequence 0 of grad_cum / proj_end row a_w + T_w ..., sequences xseq /
// pseq elements apart; rows beyond `rows` (the end of the tensor) are skipped.
// Blocks (x, b); lenw / okb of the window, (B,).
__global__ void window_halo_add_kernel(const float* thalo, const float* halo, const double* mframe,
                                       const int64_t* lenw, const int* okb, int P, int Lc, int Kmax, int C, int rows,
                                       const float* gout, float* gcum_e, float* gpe_e, int64_t xseq, int64_t pseq) {
  const int b = blockIdx.y;
  if (okb[b] == 0) return;
  const int lw = (int)lenw[b];
  const int jl = lw > 0 ? (lw - 1) / Lc : 0;
  const double g = (double)gout[b];
  const float ft = (float)(g * mframe[(size_t)b * P + jl]);
  const float fb = jl >= 1 ? (float)(g * mframe[(size_t)b * P + jl - 1]) : 0.0f;
  const int thb = jl * Lc;  // t_hi of chunk jl - 1
  const float* th = thalo + (size_t)b * Kmax * C;
  const float* hl = halo + ((size_t)b * P + (jl >= 1 ? jl - 1 : 0)) * Kmax * C;
  for (int idx = threadIdx.x + blockIdx.x * blockDim.x; idx < (Kmax - 1) * C; idx += blockDim.x * gridDim.x) {
    const int i = idx / C, c = idx % C;
    if (1 + i > rows) continue;
    float v = ft * th[idx];
    const int hr = lw + 1 + i - thb;  // halo row of chunk jl - 1
    if (jl >= 1 && hr < Kmax) v += fb * hl[(size_t)hr * C + c];
    gcum_e[(size_t)b * xseq + (size_t)(1 + i) * C + c] += v;
    if (gpe_e != nullptr) gpe_e[(size_t)b * pseq + (size_t)i * C + c] += v;
  }
}

__global__ void fill_zero_kernel(float* p, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    p[i] = 0.0f;
}

int grid_for(size_t n) {
  size_t g = (n + 255) / 256;
  return (int)(g < 1 ? 1 : (g > 4096 ? 4096 : g));
}

}  // namespace

int launch_window_setup(const int64_t* lengths, int B, int T, int Wlen, int nw, int64_t* lenw, int* okf, int* okb,
                        hipStream_t s) {
  hipLaunchKernelGGL(window_setup_kernel, dim3((B * nw + 255) / 256), dim3(256), 0, s, lengths, B, T, Wlen, nw, lenw,
                     okf, okb);
  return hipGetLastError();
}

int launch_ck_extract(const float* st_end, const double* lv_end, const double* offs, int B, int P, int Wc, int Kmax,
                      int C, int nw, float* ck_st, double* ck_lv, double* ck_al, hipStream_t s) {
  if (nw > 1) hipLaunchKernelGGL(ck_extract_kernel, dim3(nw - 1, B), dim3(256), 0, s, st_end, lv_end, offs, B, P, Wc,
                                 Kmax, C, ck_st, ck_lv, ck_al);
  return hipGetLastError();
}

int launch_window_row0(const float* ck_ah, const double* ck_al, const int* okf, int B, int Tw, int C, float* ah,
                       double* al, hipStream_t s) {
  hipLaunchKernelGGL(window_row0_kernel, dim3(B), dim3(64), 0, s, ck_ah, ck_al, okf, Tw, C, ah, al);
  return hipGetLastError();
}

int launch_window_state_fix(double* lv, const double* offs, int B, int P, int Kmax, hipStream_t s) {
  hipLaunchKernelGGL(window_state_fix_kernel, dim3(B), dim3(256), 0, s, lv, offs, P, Kmax);
  return hipGetLastError();
}

int launch_window_halo_add(const float* thalo, const float* halo, const double* mframe, const int64_t* lenw,
                           const int* okb, int B, int P, int Lc, int Kmax, int C, int rows, const float* gout,
                           float* gcum_e, float* gpe_e, int64_t xseq, int64_t pseq, hipStream_t s) {
  if (Kmax < 2) return hipSuccess;
  const int gx = std::min(grid_for((size_t)(Kmax - 1) * C), 64);
  hipLaunchKernelGGL(window_halo_add_kernel, dim3(gx, B), dim3(256), 0, s, thalo, halo, mframe, lenw, okb, P, Lc, Kmax,
                     C, rows, gout, gcum_e, gpe_e, xseq, pseq);
  return hipGetLastError();
}

int launch_fill_zero(float* p, size_t n, hipStream_t s) {
  if (p == nullptr || n == 0) return hipSuccess;
  hipLaunchKernelGGL(fill_zero_kernel, dim3(grid_for(n)), dim3(256), 0, s, p, n);
  return hipGetLastError();
}

}  // namespace tsm
