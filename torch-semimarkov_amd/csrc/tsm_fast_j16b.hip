// Register-resident scan and marginal instances: 16-lane label groups, 17-32 durations per lane.
// (Split across files so the instances compile in parallel.)
#include "tsm_fastscan.hpp"
#include "tsm_margfast.hpp"

namespace tsm {

int launch_fast_j16_hi(const Plan& pl, const ScanParams& p, bool fwd, hipStream_t st) {
  switch (pl.FR) {
    case 17: return fastscan::launch_fast_jr<16, 17>(pl, p, fwd, st);
    case 18: return fastscan::launch_fast_jr<16, 18>(pl, p, fwd, st);
    case 19: return fastscan::launch_fast_jr<16, 19>(pl, p, fwd, st);
    case 20: return fastscan::launch_fast_jr<16, 20>(pl, p, fwd, st);
    case 21: return fastscan::launch_fast_jr<16, 21>(pl, p, fwd, st);
    case 22: return fastscan::launch_fast_jr<16, 22>(pl, p, fwd, st);
    case 23: return fastscan::launch_fast_jr<16, 23>(pl, p, fwd, st);
    case 24: return fastscan::launch_fast_jr<16, 24>(pl, p, fwd, st);
    case 25: return fastscan::launch_fast_jr<16, 25>(pl, p, fwd, st);
    case 26: return fastscan::launch_fast_jr<16, 26>(pl, p, fwd, st);
    case 27: return fastscan::launch_fast_jr<16, 27>(pl, p, fwd, st);
    case 28: return fastscan::launch_fast_jr<16, 28>(pl, p, fwd, st);
    case 29: return fastscan::launch_fast_jr<16, 29>(pl, p, fwd, st);
    case 30: return fastscan::launch_fast_jr<16, 30>(pl, p, fwd, st);
    case 31: return fastscan::launch_fast_jr<16, 31>(pl, p, fwd, st);
    case 32: return fastscan::launch_fast_jr<16, 32>(pl, p, fwd, st);
    default: return (int)hipErrorInvalidValue;
  }
}

int launch_fast_j16(const Plan& pl, const ScanParams& p, bool fwd, hipStream_t st) {
  return pl.FR <= 16 ? launch_fast_j16_lo(pl, p, fwd, st) : launch_fast_j16_hi(pl, p, fwd, st);
}

int launch_margfast_j16_hi(const Plan& pl, const MargParams& q, hipStream_t st) {
  switch (pl.MR) {
    case 17: return margfast::launch_margfast_jr<16, 17>(pl, q, st);
    case 18: return margfast::launch_margfast_jr<16, 18>(pl, q, st);
    case 19: return margfast::launch_margfast_jr<16, 19>(pl, q, st);
    case 20: return margfast::launch_margfast_jr<16, 20>(pl, q, st);
    case 21: return margfast::launch_margfast_jr<16, 21>(pl, q, st);
    case 22: return margfast::launch_margfast_jr<16, 22>(pl, q, st);
    case 23: return margfast::launch_margfast_jr<16, 23>(pl, q, st);
    case 24: return margfast::launch_margfast_jr<16, 24>(pl, q, st);
    case 25: return margfast::launch_margfast_jr<16, 25>(pl, q, st);
    case 26: return margfast::launch_margfast_jr<16, 26>(pl, q, st);
    case 27: return margfast::launch_margfast_jr<16, 27>(pl, q, st);
    case 28: return margfast::launch_margfast_jr<16, 28>(pl, q, st);
    case 29: return margfast::launch_margfast_jr<16, 29>(pl, q, st);
    case 30: return margfast::launch_margfast_jr<16, 30>(pl, q, st);
    case 31: return margfast::launch_margfast_jr<16, 31>(pl, q, st);
    case 32: return margfast::launch_margfast_jr<16, 32>(pl, q, st);
    default: return (int)hipErrorInvalidValue;
  }
}

int launch_margfast_j16(const Plan& pl, const MargParams& q, hipStream_t st) {
  if (pl.C > 64) return launch_margfast_j16_wide(pl, q, st);
  return pl.MR <= 16 ? launch_margfast_j16_lo(pl, q, st) : launch_margfast_j16_hi(pl, q, st);
}

int launch_fast_max_j16_hi(const Plan& pl, const ScanParams& p, hipStream_t st) {
  switch (pl.FR) {
    case 17: return fastscan::launch_fast_max_jr<16, 17>(pl, p, st);
    case 18: return fastscan::launch_fast_max_jr<16, 18>(pl, p, st);
    case 19: return fastscan::launch_fast_max_jr<16, 19>(pl, p, st);
    case 20: return fastscan::launch_fast_max_jr<16, 20>(pl, p, st);
    case 21: return fastscan::launch_fast_max_jr<16, 21>(pl, p, st);
    case 22: return fastscan::launch_fast_max_jr<16, 22>(pl, p, st);
    case 23: return fastscan::launch_fast_max_jr<16, 23>(pl, p, st);
    case 24: return fastscan::launch_fast_max_jr<16, 24>(pl, p, st);
    case 25: return fastscan::launch_fast_max_jr<16, 25>(pl, p, st);
    case 26: return fastscan::launch_fast_max_jr<16, 26>(pl, p, st);
    case 27: return fastscan::launch_fast_max_jr<16, 27>(pl, p, st);
    case 28: return fastscan::launch_fast_max_jr<16, 28>(pl, p, st);
    case 29: return fastscan::launch_fast_max_jr<16, 29>(pl, p, st);
    case 30: return fastscan::launch_fast_max_jr<16, 30>(pl, p, st);
    case 31: return fastscan::launch_fast_max_jr<16, 31>(pl, p, st);
    case 32: return fastscan::launch_fast_max_jr<16, 32>(pl, p, st);
    default: return (int)hipErrorInvalidValue;
  }
}

int launch_fast_max_j16(const Plan& pl, const ScanParams& p, hipStream_t st) {
  return pl.FR <= 16 ? launch_fast_max_j16_lo(pl, p, st) : launch_fast_max_j16_hi(pl, p, st);
}

}  // namespace tsm
