// Launch plan shared by the host entry points and the kernels: thread
// mapping, ring sizes, LDS layout, chunking.  Every size a kernel derives from
// here is derived identically on the host, so LDS/workspace layouts agree.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace tsm {

// Per-class lane group size J (power of two <= 64): thread tid works for label
// c = tid / J on durations k = 1 + (tid % J) + J*r.  NT = round_up(C*J, 64).
struct Plan {
  int B, T, C, K, Kmax;
  int J, NT, RS;     // lanes per class, threads per block, ring length
  int P, Lc, W;      // scan chunks per sequence, chunk length, warm-up steps
  int global_rings;  // 1: rings live in the workspace (LDS too small)
  size_t scan_lds;   // dynamic LDS bytes of the scan kernels
  int NB, TB;        // marginal: position blocks per sequence, positions per block
  int CB, NCB;       // marginal: destination labels per block, label blocks
  int JM, NTM;       // marginal: lanes per label, threads per block
  size_t marg_lds;   // dynamic LDS bytes of the marginal kernel
  int has_ps, has_pe;
};

__host__ __device__ inline size_t align16(size_t x) { return (x + 15) & ~size_t(15); }

// ---- scan kernel LDS layout (bytes offsets) --------------------------------
struct ScanLds {
  size_t lring;  // double[RS]
  size_t urng;   // float[C*RS]   (ring of normalised values)   -- LDS only if !global
  size_t crng;   // float[C*RS]   (ring of cumulative scores)
  size_t prng;   // float[C*RS]   (ring of projection scores)   -- only if a projection
  size_t dbt;    // float[C*(Kmax+1)]  duration bias, log2 units, [c][k]
  size_t trt;    // float[C*C]    transition, log2 units, mix layout [class][inner]
  size_t row;    // float[2*C]    normalised row for the label mix (double buffered)
  size_t dlt;    // float[2*(Kmax+1)] level differences per duration (double buffered)
  size_t wred;   // float[2*32]   per-wave maxima (double buffered)
  size_t red;    // double[64]    block reductions (verification)
  size_t total;
};

__host__ __device__ inline ScanLds scan_lds_layout(int C, int Kmax, int RS, int has_proj, int global_rings) {
  ScanLds L;
  size_t o = 0;
  L.lring = o; o = align16(o + sizeof(double) * RS);
  L.red = o; o = align16(o + sizeof(double) * 64);
  const size_t ring = sizeof(float) * (size_t)C * RS;
  const size_t dbsz = sizeof(float) * (size_t)C * (Kmax + 1);
  if (!global_rings) {
    L.urng = o; o = align16(o + ring);
    L.crng = o; o = align16(o + ring);
    L.prng = o; o = align16(o + (has_proj ? ring : 0));
    L.dbt = o; o = align16(o + dbsz);
  } else {
    L.urng = L.crng = L.prng = L.dbt = 0;
  }
  L.trt = o; o = align16(o + sizeof(float) * (size_t)C * C);
  L.row = o; o = align16(o + sizeof(float) * 2 * C);
  L.dlt = o; o = align16(o + sizeof(float) * 2 * (Kmax + 1));
  L.wred = o; o = align16(o + sizeof(float) * 64);
  L.total = o;
  return L;
}

// Per work item global ring footprint (floats) when the rings do not fit LDS:
// urng, crng, prng (C*RS each) + dbt (C*(Kmax+1)).
__host__ __device__ inline size_t scan_gring_floats(int C, int Kmax, int RS) {
  return 3 * (size_t)C * RS + (size_t)C * (Kmax + 1);
}

// ---- marginal kernel LDS layout (one block of CB destination labels) -------
struct MargLds {
  size_t lvb;    // double[RS]      beta levels ring
  size_t brng;   // float[CB*RS]    beta-hat ring
  size_t crng;   // float[CB*RS]    cum ring
  size_t prng;   // float[CB*RS]    proj_end ring (if present)
  size_t erng;   // float[CB*RS]    end-sum accumulation ring
  size_t dbt;    // float[CB*(Kmax+1)]
  size_t dacc;   // float[CB*(Kmax+1)] duration-gradient accumulators (lane owned)
  size_t trt;    // float[CB*C]     transition [c_dst (local)][c_src], log2 units
  size_t row;    // float[2*C]      alpha-hat row (double buffered)
  size_t bk;     // float[2*(Kmax+1)] per-duration exponent offsets (double buffered)
  size_t total;
};

__host__ __device__ inline MargLds marg_lds_layout(int C, int CB, int Kmax, int RS, int has_pe) {
  MargLds L;
  size_t o = 0;
  L.lvb = o; o = align16(o + sizeof(double) * RS);
  const size_t ring = sizeof(float) * (size_t)CB * RS;
  L.brng = o; o = align16(o + ring);
  L.crng = o; o = align16(o + ring);
  L.prng = o; o = align16(o + (has_pe ? ring : 0));
  L.erng = o; o = align16(o + ring);
  L.dbt = o; o = align16(o + sizeof(float) * (size_t)CB * (Kmax + 1));
  L.dacc = o; o = align16(o + sizeof(float) * (size_t)CB * (Kmax + 1));
  L.trt = o; o = align16(o + sizeof(float) * (size_t)CB * C);
  L.row = o; o = align16(o + sizeof(float) * 2 * C);
  L.bk = o; o = align16(o + sizeof(float) * 2 * (Kmax + 1));
  L.total = o;
  return L;
}

}  // namespace tsm
