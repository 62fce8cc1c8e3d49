// Launch plan shared by the host entry points and the kernels: thread
// mapping, ring sizes, LDS layout, chunking.  Every size a kernel derives from
// here is derived identically on the host, so LDS/workspace layouts agree.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace tsm {

// Per-class lane group size J (power of two <= 64): thread tid works for label
// c = tid / J on durations k = 1 + (tid % J) + J*r, r < R = ceil(Kmax/J).
// NT = round_up(C*J, 64).  KP = J*R >= Kmax is the padded duration range.
struct Plan {
  int B, T, C, K, Kmax;
  int J, NT, RS;     // lanes per class, threads per block, ring slots (>= Kmax+2, >= KP+1)
  int R, KP, RL;     // durations per lane, padded durations, ring row length (>= RS + KP,
                     // RL % 64 == J % 64 so the label groups of a wave hit distinct banks)
  int RMAX;          // register terms per lane in the scans (32) or 0 for the generic loop
  int P, Lc, W;      // scan chunks per sequence, chunk length, warm-up steps
  int global_rings;  // 1: rings live in the workspace (LDS too small)
  size_t scan_lds;   // dynamic LDS bytes of the scan kernels
  int NB, TB;        // marginal: position blocks per sequence, positions per block
  int CB, NCB;       // marginal: destination labels per block, label blocks
  int JM, NTM;       // marginal: lanes per label, threads per block
  size_t marg_lds;   // dynamic LDS bytes of the marginal kernel
  int has_ps, has_pe;
  // register-resident log-semiring scan ("fast" path), used when fast == 1:
  // FJ lanes per label, FR durations per lane (compile-time), FNT threads,
  // FRS level slots, FRL ring length per label (fp64 entries), fast_lds bytes
  int fast, FJ, FR, FNT, FRS, FRL;
  size_t fast_lds;
  // the operand stage the fused-marginal beta scan keeps behind the rings (16-lane
  // plans): FSB steps per batch (16, 8 or 4), fstage bytes (per label group two
  // float4 per step and one of padding); 0 when it does not fit, and then the
  // marginals stay separate
  size_t fstage;
  int FSB;
  // Two chunks per CU for a fast scan direction whose compiled instance leaves
  // room for a second workgroup on every SIMD: P2 chunks of Lc2 positions per
  // sequence, rings of FRL2 entries (fast_lds2 bytes).  dualF / dualB / dualV: the
  // log forward, the log backward with separate marginals and the Viterbi
  // forward run with them; regsF / regsB / regsV: those instances' VGPRs.
  int P2, Lc2, FRL2, dualF, dualB, dualV, regsF, regsB, regsV;
  size_t fast_lds2;
  // register-resident marginal kernel (mfast == 1): 16 lanes per label, MR
  // durations per lane, one wavefront of 4 labels per workgroup, MRS level
  // slots of the generic layout, MRL linear ring length.  NB, TB, CB, NCB and
  // marg_lds above then describe its blocking.
  int mfast, MR, MRS, MRL;
  // duration-dependent (trows, C, C) transitions (trows > 0): dense scans with DJ
  // lanes per label and DNT threads, DRS ring slots, dense_lds bytes, transition
  // table in LDS when dtrl == 1; dense marginals with DG lanes per label group,
  // DNTM threads, DNB blocks of DTB start positions, dmarg_lds bytes
  int trows, dense, DJ, DNT, DRS, dtrl;
  size_t dense_lds;
  int DG, DNTM, DNB, DTB;
  size_t dmarg_lds;
  // cooperative log-semiring scan (coop == 1, tsm_coopscan.hpp) when the rings of
  // all labels do not fit one CU: groups of CG blocks, CCL labels per block with
  // 16 lanes each (CNT threads), CR durations per lane, CRS ring slots, CRL ring
  // row length, coop_lds bytes; CNQ co-resident groups, CGRID blocks, cxmap = 1
  // when members share blockIdx % 8
  int coop, CG, CCL, CR, CNT, CRS, CRL, CNQ, CGRID, cxmap;
  size_t coop_lds;
  // backward with the marginals fused into the register-resident beta scan
  // (mfused == 1; needs fast with FJ == 16): GNB transition-gradient row blocks
  // of GTB starts per sequence
  int mfused, GNB, GTB;
};



__host__ __device__ inline size_t align16(size_t x) { return (x + 15) & ~size_t(15); }

// LDS layout of the register-resident marginal kernel (one wavefront of CB
// labels): per label an fp64 x ring of RL entries, then the per-step operands
// of one batch of J positions.
struct MargFastLds {
  size_t xring;  // double[CB*RL]
  size_t alv;    // double[J]    alpha levels
  size_t cmv;    // double[CB*J] cumulative scores of the own labels (emission input: in the block's frame)
  size_t carry;  // double[CB][2] emission input: running cum of the x and step streams
  size_t psv;    // float[CB*J]  proj_start of the own labels
  size_t total;
};

__host__ __device__ inline MargFastLds margfast_lds_layout(int CB, int RL, int J, int C) {
  MargFastLds L;
  size_t o = 0;
  L.xring = o; o = align16(o + 8 * (size_t)CB * RL);
  L.alv = o; o = align16(o + 8 * (size_t)J);
  L.cmv = o; o = align16(o + 8 * (size_t)CB * J);
  L.carry = o; o = align16(o + 16 * (size_t)CB);
  L.psv = o; o = align16(o + 4 * (size_t)CB * J);
  L.total = o;
  return L;
}

// ---- dense scan LDS layout (duration-dependent transitions) ----------------
// Rings are position-major: ring slot s (position pos, s = pos % RS) holds the
// row of all C labels, so the source-label loop of one duration reads
// consecutive words.
struct DenseLds {
  size_t ring;   // float[RS*CS]    normalised state rows (alpha-hat / beta-hat), CS = C|1
  size_t crng;   // float[RS*CS]    cumulative scores of the ring positions
  size_t prng;   // float[RS*CS]    projection of the ring positions (log2 units)
  size_t lring;  // double[RS]      per-position levels
  size_t dbt;    // float[(Kmax+1)*C] duration bias, log2 units, [k][c]
  size_t wk;     // float[Kmax*CS]  backward: per-duration terms of the current step, [k-1][c]
  size_t dlt;    // float[Kmax+1]   level difference per duration (-1e30 when invalid)
  size_t wred;   // float[64]       per-wave maxima
  size_t red;    // double[64]      block reductions (verification)
  size_t trk;    // float[Kmax*C*CS] transitions, log2 units, rows [k-1][out] (only when in LDS)
  size_t total;
};

__host__ __device__ inline DenseLds dense_lds_layout(int C, int Kmax, int RS, int trl) {
  DenseLds L;
  const size_t CS = (size_t)(C | 1);  // odd row stride (LDS banks)
  size_t o = 0;
  const size_t ring = sizeof(float) * (size_t)RS * CS;
  L.ring = o; o = align16(o + ring);
  L.crng = o; o = align16(o + ring);
  L.prng = o; o = align16(o + ring);
  L.lring = o; o = align16(o + sizeof(double) * RS);
  L.dbt = o; o = align16(o + sizeof(float) * (size_t)(Kmax + 1) * C);
  L.wk = o; o = align16(o + sizeof(float) * (size_t)Kmax * CS);
  L.dlt = o; o = align16(o + sizeof(float) * (Kmax + 1));
  L.wred = o; o = align16(o + sizeof(float) * 64);
  L.red = o; o = align16(o + sizeof(double) * 64);
  L.trk = o; o = align16(o + (trl ? sizeof(float) * (size_t)Kmax * C * CS : 0));
  L.total = o;
  return L;
}

// Dense marginal kernel: start sums of the block's TB positions and end sums of
// the TB + Kmax rows its segments can end on.
struct DenseMargLds {
  size_t sacc;   // float[TB*C]
  size_t eacc;   // float[(TB+Kmax)*C]
  size_t total;
};

__host__ __device__ inline DenseMargLds dense_marg_lds_layout(int C, int Kmax, int TB) {
  DenseMargLds L;
  size_t o = 0;
  L.sacc = o; o = align16(o + sizeof(float) * (size_t)TB * C);
  L.eacc = o; o = align16(o + sizeof(float) * (size_t)(TB + Kmax) * C);
  L.total = o;
  return L;
}

// ---- fast scan LDS layout ---------------------------------------------------
// One linear ring per label of RL > KP fp64 entries (the current position one
// index below the previous one, the KP newest entries copied to the top when
// the index runs out), and the levels of the last RS positions (pos % RS).
// Entry = level + normalised state (+ folded projection) - sgn * cumulative
// score, all in log2 units.
struct FastLds {
  size_t ring;   // double[C*RL]
  size_t lring;  // double[RS]   per-position levels
  size_t row;    // float[2*C]   per-step row of all labels (double buffered)
  size_t red;    // double[64]   block reductions (verification)
  size_t stage;  // fused marginals: per-step operands of a batch of steps, stage bytes
  size_t total;
};

__host__ __device__ inline FastLds fast_lds_layout(int C, int RL, int RS, size_t stage) {
  FastLds L;
  size_t o = 0;
  L.ring = o; o = align16(o + 8 * (size_t)C * RL);
  L.lring = o; o = align16(o + sizeof(double) * RS);
  L.row = o; o = align16(o + sizeof(float) * 2 * C);
  L.red = o; o = align16(o + sizeof(double) * 64);
  L.stage = o; o = align16(o + stage);
  L.total = o;
  return L;
}

// ---- cooperative scan LDS layout (one member of a group) -------------------
// Linear rings of the member's CL labels (compacted like the fast scan's), per-position
// levels, the double-buffered row of all C labels, block reductions and the
// give-up flag.
struct CoopLds {
  size_t ring, lring, row, red, flag, total;
};

__host__ __device__ inline CoopLds coop_lds_layout(int CL, int C, int RL, int RS) {
  CoopLds L;
  size_t o = 0;
  L.ring = o; o = align16(o + 8 * (size_t)CL * RL);
  L.lring = o; o = align16(o + sizeof(double) * RS);
  L.row = o; o = align16(o + sizeof(float) * 2 * C);
  L.red = o; o = align16(o + sizeof(double) * 64);
  L.flag = o; o = align16(o + sizeof(int));
  L.total = o;
  return L;
}

// ---- scan kernel LDS layout (bytes offsets) --------------------------------
// Rings hold, per label, RL = RS + KP floats: slot s (0 <= s < RS) plus a mirror
// copy of slots s < KP at s + RS, so the KP durations of a step are read at
// consecutive indices without wrap-around.
struct ScanLds {
  size_t lring;  // double[RS]      per-position levels (log2 units)
  size_t red;    // double[64]      block reductions (verification)
  size_t urng;   // float[C*RL]     state ring (normalised values + folded projection)
  size_t crng;   // float[C*RL]     ring of cumulative scores
  size_t dbt;    // float[C*(KP+1)] duration bias, log2 units, [c][k] (generic loop only)
  size_t trt;    // float[C*C]      transition, log2 units, mix layout [class][inner]
  size_t row;    // float[C]        row for the label mix
  size_t dlt;    // float[KP+1]     level difference per duration (-1e30 when invalid)
  size_t wred;   // float[64]       per-wave maxima
  size_t total;
};

__host__ __device__ inline ScanLds scan_lds_layout(int C, int KP, int RS, int RL, int global_rings) {
  ScanLds L;
  size_t o = 0;
  L.lring = o; o = align16(o + sizeof(double) * RS);
  L.red = o; o = align16(o + sizeof(double) * 64);
  if (!global_rings) {
    L.urng = o; o = align16(o + sizeof(float) * (size_t)C * RL);
    L.crng = o; o = align16(o + sizeof(float) * (size_t)C * RL);
    L.dbt = o; o = align16(o + sizeof(float) * (size_t)C * (KP + 1));
  } else {
    L.urng = L.crng = L.dbt = 0;
  }
  L.trt = o; o = align16(o + sizeof(float) * (size_t)C * C);
  L.row = o; o = align16(o + sizeof(float) * C);
  L.dlt = o; o = align16(o + sizeof(float) * (KP + 1));
  L.wred = o; o = align16(o + sizeof(float) * 64);
  L.total = o;
  return L;
}

// Per work item ring footprint (floats) in the workspace when LDS is too small.
__host__ __device__ inline size_t scan_gring_floats(int C, int KP, int RL) {
  return 2 * (size_t)C * RL + (size_t)C * (KP + 1);
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
