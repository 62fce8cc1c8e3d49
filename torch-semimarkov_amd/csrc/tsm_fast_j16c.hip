// Register-resident marginal instances for 64 < C <= 128: eight source labels
// per lane in the label mix, durations per lane rounded up to a multiple of 4
// (padded durations carry a -1e30 duration bias and add nothing).
#include "tsm_margfast.hpp"

namespace tsm {

int launch_margfast_j16_wide(const Plan& pl, const MargParams& q, hipStream_t st) {
  switch (pl.MR) {
    case 4: return margfast::launch_margfast_jr<16, 4, 8>(pl, q, st);
    case 8: return margfast::launch_margfast_jr<16, 8, 8>(pl, q, st);
    case 12: return margfast::launch_margfast_jr<16, 12, 8>(pl, q, st);
    case 16: return margfast::launch_margfast_jr<16, 16, 8>(pl, q, st);
    case 20: return margfast::launch_margfast_jr<16, 20, 8>(pl, q, st);
    case 24: return margfast::launch_margfast_jr<16, 24, 8>(pl, q, st);
    case 28: return margfast::launch_margfast_jr<16, 28, 8>(pl, q, st);
    case 32: return margfast::launch_margfast_jr<16, 32, 8>(pl, q, st);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // namespace tsm
