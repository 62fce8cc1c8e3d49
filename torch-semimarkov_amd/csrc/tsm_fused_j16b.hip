// Backward log scan with fused segment marginals, 16-lane label groups,
// 17-32 durations per lane.  (Split across files so the instances compile in
// parallel.)
#include "tsm_fastscan.hpp"

namespace tsm {

int launch_fused_j16_hi(const Plan& pl, const ScanParams& p, hipStream_t st) {
  switch (p.R) {
    case 17: return fastscan::launch_fused_r<17>(pl, p, st);
    case 18: return fastscan::launch_fused_r<18>(pl, p, st);
    case 19: return fastscan::launch_fused_r<19>(pl, p, st);
    case 20: return fastscan::launch_fused_r<20>(pl, p, st);
    case 21: return fastscan::launch_fused_r<21>(pl, p, st);
    case 22: return fastscan::launch_fused_r<22>(pl, p, st);
    case 23: return fastscan::launch_fused_r<23>(pl, p, st);
    case 24: return fastscan::launch_fused_r<24>(pl, p, st);
    case 25: return fastscan::launch_fused_r<25>(pl, p, st);
    case 26: return fastscan::launch_fused_r<26>(pl, p, st);
    case 27: return fastscan::launch_fused_r<27>(pl, p, st);
    case 28: return fastscan::launch_fused_r<28>(pl, p, st);
    case 29: return fastscan::launch_fused_r<29>(pl, p, st);
    case 30: return fastscan::launch_fused_r<30>(pl, p, st);
    case 31: return fastscan::launch_fused_r<31>(pl, p, st);
    case 32: return fastscan::launch_fused_r<32>(pl, p, st);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace tsm
