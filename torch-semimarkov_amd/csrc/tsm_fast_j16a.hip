// Register-resident scan instances: 16-lane label groups, 1-16 durations per lane.
// (Split across files so the instances compile in parallel.)
#include "tsm_fastscan.hpp"

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

}  // namespace tsm
