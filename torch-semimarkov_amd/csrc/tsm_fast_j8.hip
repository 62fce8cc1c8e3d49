// Register-resident scan instances: 8-lane label groups.
// (Split across files so the instances compile in parallel.)
#include "tsm_fastscan.hpp"

namespace tsm {

int launch_fast_j8(const Plan& pl, const ScanParams& p, bool fwd, hipStream_t st) {
  switch (pl.FR) {
    case 1: return fastscan::launch_fast_jr<8, 1>(pl, p, fwd, st);
    case 2: return fastscan::launch_fast_jr<8, 2>(pl, p, fwd, st);
    case 3: return fastscan::launch_fast_jr<8, 3>(pl, p, fwd, st);
    case 4: return fastscan::launch_fast_jr<8, 4>(pl, p, fwd, st);
    case 5: return fastscan::launch_fast_jr<8, 5>(pl, p, fwd, st);
    case 6: return fastscan::launch_fast_jr<8, 6>(pl, p, fwd, st);
    case 7: return fastscan::launch_fast_jr<8, 7>(pl, p, fwd, st);
    case 8: return fastscan::launch_fast_jr<8, 8>(pl, p, fwd, st);
    case 9: return fastscan::launch_fast_jr<8, 9>(pl, p, fwd, st);
    case 10: return fastscan::launch_fast_jr<8, 10>(pl, p, fwd, st);
    case 11: return fastscan::launch_fast_jr<8, 11>(pl, p, fwd, st);
    case 12: return fastscan::launch_fast_jr<8, 12>(pl, p, fwd, st);
    case 13: return fastscan::launch_fast_jr<8, 13>(pl, p, fwd, st);
    case 14: return fastscan::launch_fast_jr<8, 14>(pl, p, fwd, st);
    case 15: return fastscan::launch_fast_jr<8, 15>(pl, p, fwd, st);
    case 16: return fastscan::launch_fast_jr<8, 16>(pl, p, fwd, st);
    case 20: return fastscan::launch_fast_jr<8, 20>(pl, p, fwd, st);
    case 24: return fastscan::launch_fast_jr<8, 24>(pl, p, fwd, st);
    case 28: return fastscan::launch_fast_jr<8, 28>(pl, p, fwd, st);
    case 32: return fastscan::launch_fast_jr<8, 32>(pl, p, fwd, st);
    default: return (int)hipErrorInvalidValue;
  }
}

int launch_fast_max_j8(const Plan& pl, const ScanParams& p, hipStream_t st) {
  switch (pl.FR) {
    case 1: return fastscan::launch_fast_max_jr<8, 1>(pl, p, st);
    case 2: return fastscan::launch_fast_max_jr<8, 2>(pl, p, st);
    case 3: return fastscan::launch_fast_max_jr<8, 3>(pl, p, st);
    case 4: return fastscan::launch_fast_max_jr<8, 4>(pl, p, st);
    case 5: return fastscan::launch_fast_max_jr<8, 5>(pl, p, st);
    case 6: return fastscan::launch_fast_max_jr<8, 6>(pl, p, st);
    case 7: return fastscan::launch_fast_max_jr<8, 7>(pl, p, st);
    case 8: return fastscan::launch_fast_max_jr<8, 8>(pl, p, st);
    case 9: return fastscan::launch_fast_max_jr<8, 9>(pl, p, st);
    case 10: return fastscan::launch_fast_max_jr<8, 10>(pl, p, st);
    case 11: return fastscan::launch_fast_max_jr<8, 11>(pl, p, st);
    case 12: return fastscan::launch_fast_max_jr<8, 12>(pl, p, st);
    case 13: return fastscan::launch_fast_max_jr<8, 13>(pl, p, st);
    case 14: return fastscan::launch_fast_max_jr<8, 14>(pl, p, st);
    case 15: return fastscan::launch_fast_max_jr<8, 15>(pl, p, st);
    case 16: return fastscan::launch_fast_max_jr<8, 16>(pl, p, st);
    case 20: return fastscan::launch_fast_max_jr<8, 20>(pl, p, st);
    case 24: return fastscan::launch_fast_max_jr<8, 24>(pl, p, st);
    case 28: return fastscan::launch_fast_max_jr<8, 28>(pl, p, st);
    case 32: return fastscan::launch_fast_max_jr<8, 32>(pl, p, st);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace tsm
