// Register-resident scan and marginal instances: 16-lane label groups, 1-16 durations per lane.
// (Split across files so the instances compile in parallel.)
#include "tsm_fastscan.hpp"
#include "tsm_margfast.hpp"

namespace tsm {

int launch_fast_j16_lo(const Plan& pl, const ScanParams& p, bool fwd, hipStream_t st) {
  switch (pl.FR) {
    case 1: return fastscan::launch_fast_jr<16, 1>(pl, p, fwd, st);
    case 2: return fastscan::launch_fast_jr<16, 2>(pl, p, fwd, st);
    case 3: return fastscan::launch_fast_jr<16, 3>(pl, p, fwd, st);
    case 4: return fastscan::launch_fast_jr<16, 4>(pl, p, fwd, st);
    case 5: return fastscan::launch_fast_jr<16, 5>(pl, p, fwd, st);
    case 6: return fastscan::launch_fast_jr<16, 6>(pl, p, fwd, st);
    case 7: return fastscan::launch_fast_jr<16, 7>(pl, p, fwd, st);
    case 8: return fastscan::launch_fast_jr<16, 8>(pl, p, fwd, st);
    case 9: return fastscan::launch_fast_jr<16, 9>(pl, p, fwd, st);
    case 10: return fastscan::launch_fast_jr<16, 10>(pl, p, fwd, st);
    case 11: return fastscan::launch_fast_jr<16, 11>(pl, p, fwd, st);
    case 12: return fastscan::launch_fast_jr<16, 12>(pl, p, fwd, st);
    case 13: return fastscan::launch_fast_jr<16, 13>(pl, p, fwd, st);
    case 14: return fastscan::launch_fast_jr<16, 14>(pl, p, fwd, st);
    case 15: return fastscan::launch_fast_jr<16, 15>(pl, p, fwd, st);
    case 16: return fastscan::launch_fast_jr<16, 16>(pl, p, fwd, st);
    default: return (int)hipErrorInvalidValue;
  }
}

int launch_margfast_j16_lo(const Plan& pl, const MargParams& q, hipStream_t st) {
  switch (pl.MR) {
    case 1: return margfast::launch_margfast_jr<16, 1>(pl, q, st);
    case 2: return margfast::launch_margfast_jr<16, 2>(pl, q, st);
    case 3: return margfast::launch_margfast_jr<16, 3>(pl, q, st);
    case 4: return margfast::launch_margfast_jr<16, 4>(pl, q, st);
    case 5: return margfast::launch_margfast_jr<16, 5>(pl, q, st);
    case 6: return margfast::launch_margfast_jr<16, 6>(pl, q, st);
    case 7: return margfast::launch_margfast_jr<16, 7>(pl, q, st);
    case 8: return margfast::launch_margfast_jr<16, 8>(pl, q, st);
    case 9: return margfast::launch_margfast_jr<16, 9>(pl, q, st);
    case 10: return margfast::launch_margfast_jr<16, 10>(pl, q, st);
    case 11: return margfast::launch_margfast_jr<16, 11>(pl, q, st);
    case 12: return margfast::launch_margfast_jr<16, 12>(pl, q, st);
    case 13: return margfast::launch_margfast_jr<16, 13>(pl, q, st);
    case 14: return margfast::launch_margfast_jr<16, 14>(pl, q, st);
    case 15: return margfast::launch_margfast_jr<16, 15>(pl, q, st);
    case 16: return margfast::launch_margfast_jr<16, 16>(pl, q, st);
    default: return (int)hipErrorInvalidValue;
  }
}

int launch_fast_max_j16_lo(const Plan& pl, const ScanParams& p, hipStream_t st) {
  switch (pl.FR) {
    case 1: return fastscan::launch_fast_max_jr<16, 1>(pl, p, st);
    case 2: return fastscan::launch_fast_max_jr<16, 2>(pl, p, st);
    case 3: return fastscan::launch_fast_max_jr<16, 3>(pl, p, st);
    case 4: return fastscan::launch_fast_max_jr<16, 4>(pl, p, st);
    case 5: return fastscan::launch_fast_max_jr<16, 5>(pl, p, st);
    case 6: return fastscan::launch_fast_max_jr<16, 6>(pl, p, st);
    case 7: return fastscan::launch_fast_max_jr<16, 7>(pl, p, st);
    case 8: return fastscan::launch_fast_max_jr<16, 8>(pl, p, st);
    case 9: return fastscan::launch_fast_max_jr<16, 9>(pl, p, st);
    case 10: return fastscan::launch_fast_max_jr<16, 10>(pl, p, st);
    case 11: return fastscan::launch_fast_max_jr<16, 11>(pl, p, st);
    case 12: return fastscan::launch_fast_max_jr<16, 12>(pl, p, st);
    case 13: return fastscan::launch_fast_max_jr<16, 13>(pl, p, st);
    case 14: return fastscan::launch_fast_max_jr<16, 14>(pl, p, st);
    case 15: return fastscan::launch_fast_max_jr<16, 15>(pl, p, st);
    case 16: return fastscan::launch_fast_max_jr<16, 16>(pl, p, st);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace tsm
