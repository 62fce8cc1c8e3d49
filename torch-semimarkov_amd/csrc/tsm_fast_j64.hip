// Register-resident scan instances: 64-lane label groups.
// (Split across files so the instances compile in parallel.)
#include "tsm_fastscan.hpp"

namespace tsm {

int launch_fast_j64(const Plan& pl, const ScanParams& p, bool fwd, hipStream_t st) {
  switch (pl.FR) {
    case 1: return fastscan::launch_fast_jr<64, 1>(pl, p, fwd, st);
    case 2: return fastscan::launch_fast_jr<64, 2>(pl, p, fwd, st);
    case 3: return fastscan::launch_fast_jr<64, 3>(pl, p, fwd, st);
    case 4: return fastscan::launch_fast_jr<64, 4>(pl, p, fwd, st);
    case 5: return fastscan::launch_fast_jr<64, 5>(pl, p, fwd, st);
    case 6: return fastscan::launch_fast_jr<64, 6>(pl, p, fwd, st);
    case 7: return fastscan::launch_fast_jr<64, 7>(pl, p, fwd, st);
    case 8: return fastscan::launch_fast_jr<64, 8>(pl, p, fwd, st);
    default: return (int)hipErrorInvalidValue;
  }
}

int launch_fast_max_j64(const Plan& pl, const ScanParams& p, hipStream_t st) {
  switch (pl.FR) {
    case 1: return fastscan::launch_fast_max_jr<64, 1>(pl, p, st);
    case 2: return fastscan::launch_fast_max_jr<64, 2>(pl, p, st);
    case 3: return fastscan::launch_fast_max_jr<64, 3>(pl, p, st);
    case 4: return fastscan::launch_fast_max_jr<64, 4>(pl, p, st);
    case 5: return fastscan::launch_fast_max_jr<64, 5>(pl, p, st);
    case 6: return fastscan::launch_fast_max_jr<64, 6>(pl, p, st);
    case 7: return fastscan::launch_fast_max_jr<64, 7>(pl, p, st);
    case 8: return fastscan::launch_fast_max_jr<64, 8>(pl, p, st);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace tsm
