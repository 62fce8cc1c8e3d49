// Backward log scan with fused segment marginals, 16-lane label groups,
// 1-16 durations per lane.  (Split across files so the instances compile in
// parallel.)
#include "tsm_fastscan.hpp"

namespace tsm {

int launch_fused_j16_lo(const Plan& pl, const ScanParams& p, hipStream_t st) {
  switch (p.R) {
    case 1: return fastscan::launch_fused_r<1>(pl, p, st);
    case 2: return fastscan::launch_fused_r<2>(pl, p, st);
    case 3: return fastscan::launch_fused_r<3>(pl, p, st);
    case 4: return fastscan::launch_fused_r<4>(pl, p, st);
    case 5: return fastscan::launch_fused_r<5>(pl, p, st);
    case 6: return fastscan::launch_fused_r<6>(pl, p, st);
    case 7: return fastscan::launch_fused_r<7>(pl, p, st);
    case 8: return fastscan::launch_fused_r<8>(pl, p, st);
    case 9: return fastscan::launch_fused_r<9>(pl, p, st);
    case 10: return fastscan::launch_fused_r<10>(pl, p, st);
    case 11: return fastscan::launch_fused_r<11>(pl, p, st);
    case 12: return fastscan::launch_fused_r<12>(pl, p, st);
    case 13: return fastscan::launch_fused_r<13>(pl, p, st);
    case 14: return fastscan::launch_fused_r<14>(pl, p, st);
    case 15: return fastscan::launch_fused_r<15>(pl, p, st);
    case 16: return fastscan::launch_fused_r<16>(pl, p, st);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace tsm
