// Backward (beta) scans with duration-dependent transitions: instantiations.
#include "tsm_dense_scan.hpp"

namespace tsm {
namespace dense {

int launch_dense_bwd(const Plan& pl, const ScanParams& p, int semiring, hipStream_t s) {
  return launch_dense_dir<false>(pl, p, semiring, s);
}

}  // namespace dense
}  // namespace tsm
